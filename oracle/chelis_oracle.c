/*
 * CPU oracle for the fused-DAG execution path: TEST INFRASTRUCTURE ONLY.
 * See chelis_oracle.h for who may load it and what pins each function.
 *
 * Build profile (oracle/Makefile): gcc -O2 -ffp-contract=off -fno-fast-math
 * -fopenmp, the reference C lane's pinned profile
 * (crates/chelis-backend-c/src/toolchain.rs:229-260). float and double
 * arithmetic is IEEE binary32/binary64 with round-to-nearest-even and no
 * contraction, so every expression below finalizes at its own dtype.
 *
 * Parallel loops only ever split independent output elements; no reduction
 * is reassociated (the same rule as the reference's OpenMP loops,
 * crates/chelis-backend-c/src/emit.rs:8113-8125).
 */
#include "chelis_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* CORE-MATH shims (crates/chelis-crmath/csrc/crmath_ffi.c), built into
 * oracle/_ref/libcrmath_ref.so. The non-`raw` shims canonicalize NaN. */
float chelis_crmath_ffi_expf(float);
double chelis_crmath_ffi_exp(double);
float chelis_crmath_ffi_logf(float);
double chelis_crmath_ffi_log(double);
float chelis_crmath_ffi_erfcf(float);
double chelis_crmath_ffi_erfc(double);
float chelis_crmath_ffi_tanhf(float);
double chelis_crmath_ffi_tanh(double);

/* Threads of the oracle's parallel loops (the CPU baseline's single-thread
 * run); returns the previous setting. */
int orc_set_threads(int n) {
    const int prev = omp_get_max_threads();
    omp_set_num_threads(n);
    return prev;
}

/* ------------------------------------------------------------------ */
/* [04-NUM-2] NaN finalization: crates/chelis-backend-c/src/fp_env.rs:46-52 */
static inline float nan32(float v) {
    if (isnan(v)) {
        uint32_t b = 0x7fc00000u;
        memcpy(&v, &b, 4);
    }
    return v;
}
static inline double nan64(double v) {
    if (isnan(v)) {
        uint64_t b = 0x7ff8000000000000ull;
        memcpy(&v, &b, 8);
    }
    return v;
}

/* ------------------------------------------------------------------ */
/* Keyed RNG: spec/05-risc-primitives.md [05-RNG-1] (splitmix64) and
 * [05-RNG-2] (derive / word / unit); [05-OP-69..72] key derivations;
 * crates/chelis-numeric-core/src/dtype_semantics.rs:4508-4540. */
uint64_t orc_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
static inline uint64_t rotl64(uint64_t x, unsigned r) { return (x << r) | (x >> (64u - r)); }
uint64_t orc_derive(uint64_t key, uint64_t j) { return orc_splitmix64(key ^ rotl64(orc_splitmix64(j), 29)); }
uint64_t orc_word(uint64_t key, uint64_t index) { return orc_splitmix64(key ^ rotl64(orc_splitmix64(index), 41)); }
double orc_unit(uint64_t key, uint64_t index) {
    /* The high 53 bits over 2^53: exact in binary64. */
    return (double)(orc_word(key, index) >> 11) * 0x1p-53;
}
void orc_split(uint64_t key, uint64_t out[2]) {
    out[0] = orc_derive(key, 0);
    out[1] = orc_derive(key, 1);
}
uint64_t orc_fold_in(uint64_t key, int64_t n) { return orc_derive(orc_derive(key, 2), (uint64_t)n); }
void orc_split_n(uint64_t key, int64_t n, uint64_t *out) {
    uint64_t base = orc_derive(key, 2);
    for (int64_t j = 0; j < n; ++j) out[j] = orc_derive(base, (uint64_t)j);
}
/* [05-OP-8]: f32 is one fmaf(high - low, round_f32(u), low); f64 one fma. */
void orc_uniform_like_f32(uint64_t key, float low, float high, float *out, int64_t n) {
    float span = high - low;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = nan32(fmaf(span, (float)orc_unit(key, (uint64_t)i), low));
}
void orc_uniform_like_f64(uint64_t key, double low, double high, double *out, int64_t n) {
    double span = high - low;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = nan64(fma(span, orc_unit(key, (uint64_t)i), low));
}

/* ------------------------------------------------------------------ */
float orc_expf(float x) { return chelis_crmath_ffi_expf(x); }
double orc_exp(double x) { return chelis_crmath_ffi_exp(x); }
float orc_logf(float x) { return chelis_crmath_ffi_logf(x); }
double orc_log(double x) { return chelis_crmath_ffi_log(x); }
float orc_erfcf(float x) { return chelis_crmath_ffi_erfcf(x); }
double orc_erfc(double x) { return chelis_crmath_ffi_erfc(x); }
float orc_tanhf(float x) { return chelis_crmath_ffi_tanhf(x); }
double orc_tanh(double x) { return chelis_crmath_ffi_tanh(x); }

/* ------------------------------------------------------------------ */
/* [05-OP-30] canonical adjacent-pair tree, streamed leaf by leaf.
 * Restates the C lane's CarryTree (crates/chelis-backend-c/src/emit.rs:
 * 272-283 struct, 8113-8215 push/total): a completed subtree of 2^d leaves
 * waits in level[d]; leaf i first absorbs one waiting subtree per trailing
 * one bit of i (the waiting, earlier subtree on the left); after the last
 * leaf the waiting subtrees fold lowest level (rightmost) first. An empty
 * slice is +0 with no addition; the stored total alone is NaN-finalized. */
#define DEFINE_TREE_SUM(NAME, T, NANF)                                         \
    T NAME(const T *x, int64_t n, int64_t stride) {                            \
        T level[64];                                                           \
        int64_t count = 0;                                                     \
        for (int64_t i = 0; i < n; ++i) {                                      \
            T carry = x[i * stride];                                           \
            int depth = 0;                                                     \
            for (int64_t pending = count++; pending & 1; pending >>= 1, ++depth) \
                carry = level[depth] + carry;                                  \
            level[depth] = carry;                                              \
        }                                                                      \
        T total = (T)0;                                                        \
        int found = 0, depth = 0;                                              \
        for (int64_t remaining = count; remaining; remaining >>= 1, ++depth) { \
            if (remaining & 1) {                                               \
                total = found ? level[depth] + total : level[depth];           \
                found = 1;                                                     \
            }                                                                  \
        }                                                                      \
        return NANF(total);                                                    \
    }
DEFINE_TREE_SUM(orc_tree_sum_f32, float, nan32)
DEFINE_TREE_SUM(orc_tree_sum_f64, double, nan64)

/* The same tree as spec/05-risc-primitives.md section 2.3 words it: one
 * pass per level pairs adjacent values left to right and carries an odd
 * final value unchanged. Kept as an independent restatement that pins the
 * streamed form above. */
#define DEFINE_LEVEL_SUM(NAME, T, NANF)                                        \
    T NAME(const T *x, int64_t n) {                                            \
        if (n == 0) return (T)0;                                               \
        T *work = (T *)malloc((size_t)n * sizeof(T));                          \
        memcpy(work, x, (size_t)n * sizeof(T));                                \
        int64_t len = n;                                                       \
        while (len > 1) {                                                      \
            int64_t next = 0;                                                  \
            for (int64_t i = 0; i + 1 < len; i += 2) work[next++] = work[i] + work[i + 1]; \
            if (len & 1) work[next++] = work[len - 1];                         \
            len = next;                                                        \
        }                                                                      \
        T total = work[0];                                                     \
        free(work);                                                            \
        return NANF(total);                                                    \
    }
DEFINE_LEVEL_SUM(orc_level_sum_f32, float, nan32)
DEFINE_LEVEL_SUM(orc_level_sum_f64, double, nan64)

/* [05-OP-12]: the first NaN in index order, with its stored bits; otherwise
 * the maximum, keeping the first stored representation among equals (so
 * -0 before +0 stays -0). n >= 1 (an empty axis traps before this). */
#define DEFINE_MAX_REDUCE(NAME, T)                                             \
    T NAME(const T *x, int64_t n, int64_t stride) {                            \
        T best = x[0];                                                         \
        if (isnan(best)) return best;                                          \
        for (int64_t i = 1; i < n; ++i) {                                      \
            T v = x[i * stride];                                               \
            if (isnan(v)) return v;                                            \
            if (v > best) best = v;                                            \
        }                                                                      \
        return best;                                                           \
    }
DEFINE_MAX_REDUCE(orc_max_reduce_f32, float)
DEFINE_MAX_REDUCE(orc_max_reduce_f64, double)

#define DEFINE_AXIS(NAME, T, LEAF)                                             \
    void NAME(const T *x, int64_t outer, int64_t n, int64_t inner, T *out) {   \
        _Pragma("omp parallel for collapse(2) schedule(static)")               \
        for (int64_t o = 0; o < outer; ++o)                                    \
            for (int64_t j = 0; j < inner; ++j)                                \
                out[o * inner + j] = LEAF(x + o * n * inner + j, n, inner);    \
    }
DEFINE_AXIS(orc_sum_axis_f32, float, orc_tree_sum_f32)
DEFINE_AXIS(orc_sum_axis_f64, double, orc_tree_sum_f64)
DEFINE_AXIS(orc_max_axis_f32, float, orc_max_reduce_f32)
DEFINE_AXIS(orc_max_axis_f64, double, orc_max_reduce_f64)

/* [05-OP-29] count: Bool8 leaves are exact 0/1 i64 combined by the same
 * tree with checked addition (an i64 count of at most 2^63-1 leaves cannot
 * overflow, so the tree's value is the plain number of ones). A byte other
 * than 0 or 1 is the reference device kernel's error code 1
 * (crates/chelis-backend-hip/src/kernels.rs:375-557). */
int32_t orc_count_axis(const uint8_t *x, int64_t outer, int64_t n, int64_t inner, int64_t *out) {
    int32_t error = 0;
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t j = 0; j < inner; ++j) {
            int64_t c = 0;
            for (int64_t i = 0; i < n; ++i) {
                uint8_t b = x[(o * n + i) * inner + j];
                if (b > 1) error = 1;
                c += b & 1;
            }
            out[o * inner + j] = c;
        }
    return error;
}

/* ------------------------------------------------------------------ */
/* Softmax rows: spec/05 section 4.2 and decompose_softmax
 * (crates/chelis-dag-core/src/tier2.rs:1098-1178): max_reduce, sub
 * (NaN-canonical), correctly rounded exp, canonical sum tree, div. Every
 * primitive finalizes at the row dtype. */
#define DEFINE_SOFTMAX(NAME, T, NANF, EXPF, MAXF, SUMF)                       \
    void NAME(const T *x, T *y, int64_t rows, int64_t n) {                     \
        _Pragma("omp parallel for schedule(static)")                           \
        for (int64_t r = 0; r < rows; ++r) {                                   \
            const T *xr = x + r * n;                                           \
            T *yr = y + r * n;                                                 \
            T m = MAXF(xr, n, 1);                                              \
            for (int64_t i = 0; i < n; ++i) yr[i] = EXPF(NANF(xr[i] - m));     \
            T s = SUMF(yr, n, 1);                                              \
            for (int64_t i = 0; i < n; ++i) yr[i] = NANF(yr[i] / s);           \
        }                                                                      \
    }
DEFINE_SOFTMAX(orc_softmax_rows_f32, float, nan32, orc_expf, orc_max_reduce_f32, orc_tree_sum_f32)
DEFINE_SOFTMAX(orc_softmax_rows_f64, double, nan64, orc_exp, orc_max_reduce_f64, orc_tree_sum_f64)

/* Softmax adjoint rows: dx = y * (g - sum(g * y))
 * (crates/chelis-dag-core/src/grad.rs:2248-2290): Mul, tree Sum, Sub, Mul. */
#define DEFINE_SOFTMAX_ADJ(NAME, T, NANF, SUMF)                                \
    void NAME(const T *y, const T *g, T *dx, int64_t rows, int64_t n) {        \
        _Pragma("omp parallel for schedule(static)")                           \
        for (int64_t r = 0; r < rows; ++r) {                                   \
            const T *yr = y + r * n, *gr = g + r * n;                          \
            T *t = (T *)malloc((size_t)(n ? n : 1) * sizeof(T));               \
            for (int64_t i = 0; i < n; ++i) t[i] = NANF(gr[i] * yr[i]);        \
            T s = SUMF(t, n, 1);                                               \
            for (int64_t i = 0; i < n; ++i) dx[r * n + i] = NANF(yr[i] * NANF(gr[i] - s)); \
            free(t);                                                           \
        }                                                                      \
    }
DEFINE_SOFTMAX_ADJ(orc_softmax_adjoint_rows_f32, float, nan32, orc_tree_sum_f32)
DEFINE_SOFTMAX_ADJ(orc_softmax_adjoint_rows_f64, double, nan64, orc_tree_sum_f64)

/* Layer norm over the last axis: spec/05 section 4.4, lower_layer_norm
 * (tier2.rs:1248-1360) with mean = tree sum / extent ([05-OP-11],
 * lower_mean tier2.rs:1183). */
#define DEFINE_LAYER_NORM(NAME, T, NANF, SUMF, SQRTF)                         \
    void NAME(const T *x, const T *gamma, const T *beta, T eps, T *y, int64_t rows, int64_t n) { \
        T extent = (T)n;                                                       \
        _Pragma("omp parallel for schedule(static)")                           \
        for (int64_t r = 0; r < rows; ++r) {                                   \
            const T *xr = x + r * n;                                           \
            T *yr = y + r * n;                                                 \
            T *c = (T *)malloc((size_t)n * sizeof(T));                         \
            T *sq = (T *)malloc((size_t)n * sizeof(T));                        \
            T mean = NANF(SUMF(xr, n, 1) / extent);                            \
            for (int64_t i = 0; i < n; ++i) {                                  \
                c[i] = NANF(xr[i] - mean);                                     \
                sq[i] = NANF(c[i] * c[i]);                                     \
            }                                                                  \
            T var = NANF(SUMF(sq, n, 1) / extent);                             \
            T denom = NANF(SQRTF(NANF(var + eps)));                            \
            for (int64_t i = 0; i < n; ++i) {                                  \
                T normed = NANF(c[i] / denom);                                 \
                T scaled = NANF(normed * gamma[i]);                            \
                yr[i] = NANF(scaled + beta[i]);                                \
            }                                                                  \
            free(c);                                                           \
            free(sq);                                                          \
        }                                                                      \
    }
DEFINE_LAYER_NORM(orc_layer_norm_rows_f32, float, nan32, orc_tree_sum_f32, sqrtf)
DEFINE_LAYER_NORM(orc_layer_norm_rows_f64, double, nan64, orc_tree_sum_f64, sqrt)

/* ------------------------------------------------------------------ */
/* GELU = mul(m(x), Phi(x)) with spec/05 section 3.3's exact Phi graph and
 * its constants (crates/chelis-numeric-core/src/activation.rs:25-56):
 * c = 1/sqrt(2), cl = 1/sqrt(2) - c, k = 2/sqrt(pi) (each rounded to the
 * dtype), Veltkamp splitter s, range bound L = 64. m(x) is the multiplicand
 * guard where(cmplt(x, lowest), -0.0, x). Every primitive is NaN-final. */
#define DEFINE_GELU(NAME, T, NANF, ERFCF, EXPF, FABS, C, CL, K, S, LOWEST)   \
    static inline T NAME##_one(T x) {                                          \
        const T c = C, cl = CL, k = K, s = S, L = (T)64, half = (T)0.5;        \
        T e = ERFCF(NANF(NANF(-x) * c));                                       \
        T z = (FABS(x) < L) ? x : (T)0;                                        \
        T a = NANF(-z);                                                        \
        T th = NANF(a * c);                                                    \
        T ta = NANF(s * a);                                                    \
        T ah = NANF(ta - NANF(ta - a));                                        \
        T al = NANF(a - ah);                                                   \
        T tc = NANF(s * c);                                                    \
        T ch = NANF(tc - NANF(tc - c));                                        \
        T cr = NANF(c - ch);                                                   \
        T t0 = NANF(NANF(ah * ch) - th);                                       \
        T t1 = NANF(t0 + NANF(ah * cr));                                       \
        T t2 = NANF(t1 + NANF(al * ch));                                       \
        T t3 = NANF(t2 + NANF(al * cr));                                       \
        T tl = NANF(t3 + NANF(a * cl));                                        \
        T g = EXPF(NANF(-NANF(th * th)));                                      \
        T corr = NANF(NANF(k * g) * tl);                                       \
        T phi = NANF(half * NANF(e - corr));                                   \
        T m = (x < LOWEST) ? (T)-0.0 : x;                                      \
        return NANF(m * phi);                                                  \
    }                                                                          \
    void NAME(const T *x, T *y, int64_t n) {                                   \
        _Pragma("omp parallel for schedule(static)")                           \
        for (int64_t i = 0; i < n; ++i) y[i] = NAME##_one(x[i]);               \
    }
DEFINE_GELU(orc_gelu_f32, float, nan32, orc_erfcf, orc_expf, fabsf, (float)0.70710678118654752440,
            (float)1.2101617485882343e-8, (float)1.12837916709551257390, 4097.0f, -3.4028234663852886e38f)
DEFINE_GELU(orc_gelu_f64, double, nan64, orc_erfc, orc_exp, fabs, 0.70710678118654752440,
            -4.833646656726457e-17, 1.12837916709551257390, 134217729.0, -1.7976931348623157e308)

/* [05-OP-43] relu = max_elem(x, +0) keeping lhs on ties and NaN bits:
 * x < 0 ? +0 : x. Its adjoint is g where cmplt(0, x), else +0
 * (crates/chelis-backend-hip/src/kernels.rs:1136-1196). */
void orc_relu_f32(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] < 0.0f ? 0.0f : x[i];
}
void orc_relu_adjoint_f32(const float *x, const float *g, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = 0.0f < x[i] ? g[i] : 0.0f;
}

/* bfloat16 and IEEE binary16 storage ([04-NUM-8]): widening is exact,
 * narrowing rounds to nearest even (overflow to infinity, binary16
 * subnormals kept) and stores NaN as the format's canonical quiet NaN
 * (crates/chelis-runtime/include/chelis_runtime.h:664-760: bf16 to f32 by a
 * 16-bit shift, f32 to bf16 by the round-half-even bias on the low half,
 * f16 through its field decomposition). */
static float orc_dec16(int kind, uint16_t h) {
    uint32_t bits;
    if (kind == 0) {
        bits = (uint32_t)h << 16;
    } else {
        const uint32_t sign = (uint32_t)(h >> 15) << 31;
        const int e = (h >> 10) & 31;
        const uint32_t m = h & 1023u;
        if (e == 31) {
            bits = sign | 0x7f800000u | (m << 13);
        } else if (e > 0) {
            bits = sign | ((uint32_t)(e - 15 + 127) << 23) | (m << 13);
        } else {
            float mag = ldexpf((float)m, -24);
            memcpy(&bits, &mag, 4);
            bits |= sign;
        }
    }
    float v;
    memcpy(&v, &bits, 4);
    return v;
}
static uint16_t orc_enc16(int kind, float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    const int nan = (b & 0x7fffffffu) > 0x7f800000u;
    if (kind == 0) {
        if (nan) return 0x7fc0u;
        const uint32_t low = b & 0xffffu, up = b >> 16;
        /* round half to even on the discarded half word */
        const uint32_t r = (low > 0x8000u || (low == 0x8000u && (up & 1u))) ? up + 1u : up;
        return (uint16_t)r;
    }
    if (nan) return 0x7e00u;
    const uint16_t sign = (uint16_t)((b >> 31) << 15);
    const int be = (int)((b >> 23) & 0xffu);
    if (be == 0xff) return (uint16_t)(sign | 0x7c00u);
    /* |v| = sig * 2^(ex) with a 24-bit integer significand */
    const uint32_t sig = be ? ((b & 0x7fffffu) | 0x800000u) : (b & 0x7fffffu);
    const int ex = (be ? be : 1) - 150;
    /* binary16 quantum at |v|: 2^-24 below 2^-14, else 2^(e - 10) */
    int q = -24;
    if (sig) {
        int top = ex + 23; /* exponent of the leading bit */
        while (top > ex && !((sig >> (top - ex)) & 1u)) --top;
        if (top - 10 > q) q = top - 10;
    }
    uint64_t kept;
    if (q <= ex) {
        kept = (uint64_t)sig << (ex - q);
    } else {
        const int sh = q - ex;
        if (sh > 40) {
            kept = 0;
        } else {
            kept = (uint64_t)sig >> sh;
            const uint64_t dropped = (uint64_t)sig & ((1ull << sh) - 1ull), half = 1ull << (sh - 1);
            if (dropped > half || (dropped == half && (kept & 1u))) ++kept;
        }
    }
    /* kept * 2^q with q >= -24: encode (a carry past 11 bits bumps q) */
    if (kept >= 2048u) {
        kept >>= 1;
        ++q;
    }
    if (kept < 1024u) return (uint16_t)(sign | kept); /* subnormal (q = -24) */
    const int e16 = q + 10 + 15;
    if (e16 >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | (kept & 1023u));
}
void orc_narrow_decode(int kind, const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_dec16(kind, x[i]);
}
void orc_narrow_encode(int kind, const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_enc16(kind, x[i]);
}
void orc_narrow_sub(int kind, const uint16_t *a, const uint16_t *b, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_enc16(kind, orc_dec16(kind, a[i]) - orc_dec16(kind, b[i]));
}
/* [05-OP-40] selections keep the chosen operand's stored bits: the left one
 * when it is NaN, or when the right is not NaN and left >= right (max) /
 * left <= right (min) (crates/chelis-backend-hip/src/kernels.rs:2291-2305). */
void orc_narrow_max(int kind, const uint16_t *a, const uint16_t *b, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float l = orc_dec16(kind, a[i]), r = orc_dec16(kind, b[i]);
        y[i] = (isnan(l) || (!isnan(r) && l >= r)) ? a[i] : b[i];
    }
}
void orc_narrow_min(int kind, const uint16_t *a, const uint16_t *b, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float l = orc_dec16(kind, a[i]), r = orc_dec16(kind, b[i]);
        y[i] = (isnan(l) || (!isnan(r) && l <= r)) ? a[i] : b[i];
    }
}
/* [05-OP-43] on stored bits: a negative, nonzero, non-NaN x gives +0, any
 * other x itself; the adjoint keeps g where x is positive, nonzero and not
 * NaN (crates/chelis-backend-hip/src/kernels.rs:1196-1260). */
void orc_narrow_relu(int kind, const uint16_t *x, uint16_t *y, int64_t n) {
    const uint16_t em = kind == 0 ? 0x7f80u : 0x7c00u, fm = kind == 0 ? 0x007fu : 0x03ffu;
    for (int64_t i = 0; i < n; ++i) {
        const uint16_t v = x[i];
        const int is_nan = (v & em) == em && (v & fm);
        y[i] = ((v & 0x8000u) && (v & 0x7fffu) && !is_nan) ? 0 : v;
    }
}
void orc_narrow_relu_adjoint(int kind, const uint16_t *x, const uint16_t *g, uint16_t *y, int64_t n) {
    const uint16_t em = kind == 0 ? 0x7f80u : 0x7c00u, fm = kind == 0 ? 0x007fu : 0x03ffu;
    for (int64_t i = 0; i < n; ++i) {
        const uint16_t v = x[i];
        const int is_nan = (v & em) == em && (v & fm);
        y[i] = (!(v & 0x8000u) && (v & 0x7fffu) && !is_nan) ? g[i] : 0;
    }
}
/* spec/04 section 5.7.1: a bf16/f16 matmul accumulates at binary32; the C
 * lane decodes, runs the binary32 canonical-tree product (each product of
 * two 16-bit values is exact in binary32) and encodes the result. */
void orc_matmul_narrow(int kind, const uint16_t *A, const uint16_t *B, uint16_t *C, int64_t M, int64_t N,
                       int64_t K) {
    float *a = malloc(sizeof(float) * (size_t)(M * K + 1)), *b = malloc(sizeof(float) * (size_t)(K * N + 1));
    float *c = malloc(sizeof(float) * (size_t)(M * N + 1));
    orc_narrow_decode(kind, A, a, M * K);
    orc_narrow_decode(kind, B, b, K * N);
    orc_matmul_f32(a, K, 1, b, N, 1, c, M, N, K);
    orc_narrow_encode(kind, c, C, M * N);
    free(a);
    free(b);
    free(c);
}

/* ProdReduce: `float acc = 1.0f; acc *= x[...]` per output in axis order,
 * then the stored value NaN-finalized (crates/chelis-backend-c/src/emit.rs:
 * 2551-2561 -> emit_reduce_simple 8817-8912). */
#define DEFINE_PROD_AXIS(NAME, T, NANF)                                          \
    void NAME(const T *x, int64_t outer, int64_t n, int64_t inner, T *out) {     \
        _Pragma("omp parallel for collapse(2) schedule(static)")                  \
        for (int64_t o = 0; o < outer; ++o)                                      \
            for (int64_t j = 0; j < inner; ++j) {                                \
                T acc = (T)1;                                                    \
                for (int64_t k = 0; k < n; ++k) acc *= x[(o * n + k) * inner + j]; \
                out[o * inner + j] = NANF(acc);                                  \
            }                                                                    \
    }
DEFINE_PROD_AXIS(orc_prod_axis_f32, float, nan32)
DEFINE_PROD_AXIS(orc_prod_axis_f64, double, nan64)

/* [05-OP-37] keyed dropout at f32: the f32-rounded unit of word(key, i) is
 * compared with the rate; a dropped element is +0, a kept one
 * x / (1 - rate) (crates/chelis-backend-c/src/emit.rs:6139-6220). The
 * replay adjoint reuses the same mask on the cotangent. */
void orc_dropout_f32(uint64_t key, const float *x, float rate, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        y[i] = (float)orc_unit(key, (uint64_t)i) < rate ? 0.0f : nan32(x[i] / (1.0f - rate));
}
void orc_dropout_replay_f32(uint64_t key, const float *g, float rate, float *dx, int64_t n) {
    orc_dropout_f32(key, g, rate, dx, n);
}
void orc_dropout_f64(uint64_t key, const double *x, double rate, double *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        y[i] = orc_unit(key, (uint64_t)i) < rate ? 0.0 : nan64(x[i] / (1.0 - rate));
}
void orc_dropout_replay_f64(uint64_t key, const double *g, double rate, double *dx, int64_t n) {
    orc_dropout_f64(key, g, rate, dx, n);
}

/* ------------------------------------------------------------------ */
/* Canonical-tree matmul: spec/05 section 4.1 (insert, mul, sum over k with
 * [05-OP-30]'s tree), which the C lane emits as an inlined product
 * (crates/chelis-backend-c/src/emit.rs:8431-8560). Each product finalizes at
 * the dtype; the k leaves of every output enter its own carry tree.
 *
 * Lanes: VL consecutive output columns and RB rows share one leaf count, so
 * their trees advance together; each lane still owns a private tree, so the
 * bits equal the one-output-at-a-time tree. */
#define DEFINE_MATMUL(NAME, T, NANF, VL)                                              \
    typedef T NAME##_vec __attribute__((vector_size(VL * sizeof(T))));                \
    void NAME(const T *A, int64_t sa0, int64_t sa1, const T *B, int64_t sb0,          \
              int64_t sb1, T *C, int64_t M, int64_t N, int64_t K) {                   \
        enum { RB = 4 };                                                              \
        int64_t rblocks = (M + RB - 1) / RB, cblocks = (N + VL - 1) / VL;             \
        _Pragma("omp parallel for collapse(2) schedule(dynamic, 4)")                  \
        for (int64_t rb = 0; rb < rblocks; ++rb)                                      \
            for (int64_t cb = 0; cb < cblocks; ++cb) {                                \
                NAME##_vec level[RB][64];                                             \
                int64_t i0 = rb * RB, j0 = cb * VL;                                   \
                int rows = (int)(M - i0 < RB ? M - i0 : RB);                          \
                int lanes = (int)(N - j0 < VL ? N - j0 : VL);                         \
                for (int64_t k = 0; k < K; ++k) {                                     \
                    NAME##_vec bv;                                                    \
                    for (int l = 0; l < VL; ++l)                                      \
                        bv[l] = l < lanes ? B[k * sb0 + (j0 + l) * sb1] : (T)0;       \
                    int trailing = 0;                                                 \
                    for (int64_t p = k; p & 1; p >>= 1) ++trailing;                   \
                    for (int r = 0; r < rows; ++r) {                                  \
                        NAME##_vec carry = A[(i0 + r) * sa0 + k * sa1] * bv;          \
                        for (int d = 0; d < trailing; ++d) carry = level[r][d] + carry; \
                        level[r][trailing] = carry;                                   \
                    }                                                                 \
                }                                                                     \
                for (int r = 0; r < rows; ++r) {                                      \
                    NAME##_vec total = {0};                                           \
                    int found = 0, depth = 0;                                         \
                    for (int64_t rem = K; rem; rem >>= 1, ++depth)                    \
                        if (rem & 1) {                                                \
                            total = found ? level[r][depth] + total : level[r][depth]; \
                            found = 1;                                                \
                        }                                                             \
                    for (int l = 0; l < lanes; ++l)                                   \
                        C[(i0 + r) * N + j0 + l] = NANF(total[l]);                    \
                }                                                                     \
            }                                                                         \
    }
DEFINE_MATMUL(orc_matmul_f32, float, nan32, 8)
DEFINE_MATMUL(orc_matmul_f64, double, nan64, 4)

/* ------------------------------------------------------------------ */
/* Configuration 1, the linear-regression gradient step (linreg.ch form):
 *   r = matmul(X, w) - y;  grad = matmul(X^T, r) / n;  loss = mean(r * r).
 * Every matmul is the canonical tree, every mean a tree sum / extent. */
void orc_linreg_step_f64(const double *X, const double *w, const double *y, double *grad,
                         double *loss, int64_t n, int64_t d) {
    double *r = (double *)malloc((size_t)n * sizeof(double));
    double *sq = (double *)malloc((size_t)n * sizeof(double));
    double *gs = (double *)malloc((size_t)d * sizeof(double));
    orc_matmul_f64(X, d, 1, w, 1, 1, r, n, 1, d);
    for (int64_t i = 0; i < n; ++i) {
        r[i] = nan64(r[i] - y[i]);
        sq[i] = nan64(r[i] * r[i]);
    }
    orc_matmul_f64(X, 1, d, r, 1, 1, gs, d, 1, n);
    double extent = (double)n;
    for (int64_t k = 0; k < d; ++k) grad[k] = nan64(gs[k] / extent);
    *loss = nan64(orc_tree_sum_f64(sq, n, 1) / extent);
    free(r);
    free(sq);
    free(gs);
}

/* ------------------------------------------------------------------ */
static float *falloc(int64_t n) { return (float *)malloc((size_t)n * sizeof(float)); }

/* y[rows, n] = matmul(x, W) + insert(b, 0, rows) */
static void linear_f32(const float *x, const float *W, const float *b, float *y, int64_t rows,
                       int64_t k, int64_t n) {
    orc_matmul_f32(x, k, 1, W, n, 1, y, rows, n, k);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < n; ++j) y[i * n + j] = nan32(y[i * n + j] + b[j]);
}

/* Configuration 4: one pre-LN transformer block, causal multi-head
 * attention (spec/05 section 4.7) and a GELU FFN, all f32:
 *   h = LN1(x); q,k,v = linear(h); per head: s = (q k^T) * scale,
 *   masked = where(j <= i, s, -inf), p = softmax(masked), o = p v;
 *   x1 = x + linear_o(o); y = x1 + linear_2(GELU(linear_1(LN2(x1)))).
 * params: ln1_g ln1_b Wq bq Wk bk Wv bv Wo bo ln2_g ln2_b W1 b1 W2 b2. */
void orc_transformer_block_f32(const float *x, const float *const *P, float *out, int64_t batch,
                               int64_t seq, int64_t dm, int64_t heads, int64_t ffn) {
    int64_t rows = batch * seq, dh = dm / heads;
    const float eps = 1e-5f;
    const float scale = 1.0f / sqrtf((float)dh);
    float *h = falloc(rows * dm), *q = falloc(rows * dm), *k = falloc(rows * dm);
    float *v = falloc(rows * dm), *o = falloc(rows * dm), *x1 = falloc(rows * dm);
    float *f = falloc(rows * ffn), *sc = falloc(seq * seq);
    orc_layer_norm_rows_f32(x, P[0], P[1], eps, h, rows, dm);
    linear_f32(h, P[2], P[3], q, rows, dm, dm);
    linear_f32(h, P[4], P[5], k, rows, dm, dm);
    linear_f32(h, P[6], P[7], v, rows, dm, dm);
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t hd = 0; hd < heads; ++hd) {
            const float *qb = q + b * seq * dm + hd * dh;
            const float *kb = k + b * seq * dm + hd * dh;
            const float *vb = v + b * seq * dm + hd * dh;
            orc_matmul_f32(qb, dm, 1, kb, 1, dm, sc, seq, seq, dh);
            for (int64_t i = 0; i < seq; ++i)
                for (int64_t j = 0; j < seq; ++j) {
                    float s = nan32(sc[i * seq + j] * scale);
                    sc[i * seq + j] = j <= i ? s : -INFINITY;
                }
            orc_softmax_rows_f32(sc, sc, seq, seq);
            float *ob = falloc(seq * dh);
            orc_matmul_f32(sc, seq, 1, vb, dm, 1, ob, seq, dh, seq);
            for (int64_t i = 0; i < seq; ++i)
                memcpy(o + (b * seq + i) * dm + hd * dh, ob + i * dh, (size_t)dh * sizeof(float));
            free(ob);
        }
    linear_f32(o, P[8], P[9], q, rows, dm, dm); /* q reused as the attention output */
    for (int64_t i = 0; i < rows * dm; ++i) x1[i] = nan32(x[i] + q[i]);
    orc_layer_norm_rows_f32(x1, P[10], P[11], eps, h, rows, dm);
    linear_f32(h, P[12], P[13], f, rows, dm, ffn);
    orc_gelu_f32(f, f, rows * ffn);
    linear_f32(f, P[14], P[15], q, rows, ffn, dm);
    for (int64_t i = 0; i < rows * dm; ++i) out[i] = nan32(x1[i] + q[i]);
    free(h); free(q); free(k); free(v); free(o); free(x1); free(f); free(sc);
}

/* Configuration 5: one MLP training step (mnist.ch form) with keyed dropout:
 *   z1 = x W1 + b1; h = relu(z1); d = dropout(key, h, rate);
 *   z2 = d W2 + b2; p = softmax(z2); loss = mean(-sum(log(p) * onehot, 1));
 * reverse mode by the spec's adjoints (mean: g / extent; neg; sum: expand;
 * mul; log: g / x; softmax: y * (g - sum(g * y)) as in
 * crates/chelis-dag-core/src/grad.rs:2248; matmul: the transposed
 * canonical-tree contractions; bias: tree sum over the batch; dropout
 * replay; relu adjoint), then SGD w = w - lr * g in place. */
void orc_mlp_train_step_f32(const float *x, const float *onehot, float *w1, float *b1, float *w2,
                            float *b2, uint64_t key, float rate, float lr, float *loss,
                            int64_t B, int64_t din, int64_t dh, int64_t dout) {
    float *z1 = falloc(B * dh), *hd = falloc(B * dh), *d = falloc(B * dh);
    float *z2 = falloc(B * dout), *p = falloc(B * dout), *t = falloc(B * dout);
    float *nl = falloc(B), *gz2 = falloc(B * dout), *gd = falloc(B * dh);
    float *gw2 = falloc(dh * dout), *gw1 = falloc(din * dh), *gb1 = falloc(dh), *gb2 = falloc(dout);
    if (dout > 64) abort(); /* the per-row softmax-adjoint scratch below holds 64 classes */
    linear_f32(x, w1, b1, z1, B, din, dh);
    orc_relu_f32(z1, hd, B * dh);
    orc_dropout_f32(key, hd, rate, d, B * dh);
    linear_f32(d, w2, b2, z2, B, dh, dout);
    orc_softmax_rows_f32(z2, p, B, dout);
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t c = 0; c < dout; ++c) t[b * dout + c] = nan32(orc_logf(p[b * dout + c]) * onehot[b * dout + c]);
        nl[b] = nan32(-orc_tree_sum_f32(t + b * dout, dout, 1));
    }
    *loss = nan32(orc_tree_sum_f32(nl, B, 1) / (float)B);
    /* backward */
    float g_nl = nan32(1.0f / (float)B);
    float g_pr = nan32(-g_nl);
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t c = 0; c < dout; ++c) {
            float g_lp = nan32(g_pr * onehot[b * dout + c]);
            float g_p = nan32(g_lp / p[b * dout + c]);
            t[b * dout + c] = g_p;                    /* g */
        }
        float gy[64];
        for (int64_t c = 0; c < dout; ++c) gy[c] = nan32(t[b * dout + c] * p[b * dout + c]);
        float s = orc_tree_sum_f32(gy, dout, 1);
        for (int64_t c = 0; c < dout; ++c)
            gz2[b * dout + c] = nan32(p[b * dout + c] * nan32(t[b * dout + c] - s));
    }
    orc_sum_axis_f32(gz2, 1, B, dout, gb2);
    orc_matmul_f32(d, 1, dh, gz2, dout, 1, gw2, dh, dout, B);   /* d^T gz2 */
    orc_matmul_f32(gz2, dout, 1, w2, 1, dout, gd, B, dh, dout); /* gz2 W2^T */
    orc_dropout_replay_f32(key, gd, rate, gd, B * dh);
    orc_relu_adjoint_f32(z1, gd, gd, B * dh);
    orc_sum_axis_f32(gd, 1, B, dh, gb1);
    orc_matmul_f32(x, 1, din, gd, dh, 1, gw1, din, dh, B);      /* x^T gz1 */
    for (int64_t i = 0; i < din * dh; ++i) w1[i] = nan32(w1[i] - nan32(lr * gw1[i]));
    for (int64_t i = 0; i < dh; ++i) b1[i] = nan32(b1[i] - nan32(lr * gb1[i]));
    for (int64_t i = 0; i < dh * dout; ++i) w2[i] = nan32(w2[i] - nan32(lr * gw2[i]));
    for (int64_t i = 0; i < dout; ++i) b2[i] = nan32(b2[i] - nan32(lr * gb2[i]));
    free(z1); free(hd); free(d); free(z2); free(p); free(t); free(nl); free(gz2); free(gd);
    free(gw2); free(gw1); free(gb1); free(gb2);
}

/* ------------------------------------------------------------------ */
/* Comparison, logical, where, checked cast, checked integer arithmetic
 * and gather: the region kinds of the reference HIP lane around the float
 * path (crates/chelis-backend-hip/src/kernels.rs:1270-1346 comparison /
 * logical / where, :1382 and emit.rs:2413 casts, :769-866 and :1434 the
 * trapping integer kernels, :2557-2600 gather), restated with the C lane's
 * and the numeric core's semantics where the two lanes differ (the C lane
 * checks add and mul; the HIP lane's add and mul kernels do not).
 *
 * Dtype ids are the device packet's (chelis_runtime_dtype.h): F32 0, F64 1,
 * I32 2, BOOL 3, I64 4, BF16 5, F16 6, I8 7, I16 8. A trapping function
 * returns the row-major index of its first failing element ([04-NUM-15]),
 * or -1, and stores the failure kind of [04-NUM-9] in *kind (1 overflow,
 * 2 domain, 3 division by zero); a failing element's output is zero. */
enum { ODT_F32 = 0, ODT_F64 = 1, ODT_I32 = 2, ODT_BOOL = 3, ODT_I64 = 4, ODT_BF16 = 5, ODT_F16 = 6, ODT_I8 = 7,
       ODT_I16 = 8 };
enum { OFAIL_OVERFLOW = 1, OFAIL_DOMAIN = 2, OFAIL_DIVZERO = 3 };

static int odt_is_float(int dt) { return dt == ODT_F32 || dt == ODT_F64 || dt == ODT_BF16 || dt == ODT_F16; }
static int odt_width(int dt) {
    switch (dt) {
        case ODT_F64: case ODT_I64: return 8;
        case ODT_F32: case ODT_I32: return 4;
        case ODT_BF16: case ODT_F16: case ODT_I16: return 2;
        default: return 1;
    }
}
static int odt_bits(int dt) { return 8 * odt_width(dt); }
static void odt_limits(int dt, int64_t *lo, int64_t *hi) {
    const int b = odt_bits(dt);
    *hi = b == 64 ? INT64_MAX : (int64_t)((1ull << (b - 1)) - 1ull);
    *lo = -*hi - 1;
}

/* Element i of a float buffer widened exactly to binary64. */
static double odt_float_at(int dt, const void *p, int64_t i) {
    switch (dt) {
        case ODT_F32: return (double)((const float *)p)[i];
        case ODT_F64: return ((const double *)p)[i];
        case ODT_BF16: return (double)orc_dec16(0, ((const uint16_t *)p)[i]);
        default: return (double)orc_dec16(1, ((const uint16_t *)p)[i]);
    }
}
/* Element i of an integer or bool buffer as its exact value. */
static int64_t odt_int_at(int dt, const void *p, int64_t i) {
    switch (dt) {
        case ODT_I8: return ((const int8_t *)p)[i];
        case ODT_I16: return ((const int16_t *)p)[i];
        case ODT_I32: return ((const int32_t *)p)[i];
        case ODT_I64: return ((const int64_t *)p)[i];
        default: return ((const uint8_t *)p)[i];
    }
}
static void odt_int_store(int dt, void *p, int64_t i, int64_t v) {
    switch (dt) {
        case ODT_I8: ((int8_t *)p)[i] = (int8_t)v; break;
        case ODT_I16: ((int16_t *)p)[i] = (int16_t)v; break;
        case ODT_I32: ((int32_t *)p)[i] = (int32_t)v; break;
        case ODT_I64: ((int64_t *)p)[i] = v; break;
        default: ((uint8_t *)p)[i] = (uint8_t)v; break;
    }
}

/* [05-OP-36]: IEEE comparison of the semantic values (bf16 / f16 widened,
 * signed zeros equal, any NaN false except for neq); integers by exact
 * order; bool equality on the stored byte. kind: 0 cmplt, 1 lt, 2 eq,
 * 3 neq, 4 gt, 5 gte, 6 lte (ComparisonKind's order,
 * crates/chelis-dag-core/src/dag.rs:528-536). */
void orc_compare(int kind, int dt, const void *a, const void *b, uint8_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        int r;
        if (odt_is_float(dt)) {
            const double x = odt_float_at(dt, a, i), y = odt_float_at(dt, b, i);
            switch (kind) {
                case 0: case 1: r = x < y; break;
                case 2: r = x == y; break;
                case 3: r = x != y; break;
                case 4: r = x > y; break;
                case 5: r = x >= y; break;
                default: r = x <= y; break;
            }
        } else {
            const int64_t x = odt_int_at(dt, a, i), y = odt_int_at(dt, b, i);
            switch (kind) {
                case 0: case 1: r = x < y; break;
                case 2: r = x == y; break;
                case 3: r = x != y; break;
                case 4: r = x > y; break;
                case 5: r = x >= y; break;
                default: r = x <= y; break;
            }
        }
        out[i] = (uint8_t)r;
    }
}

/* [05-OP-26..28] on Bool8 bytes as the HIP lane reads them (a byte is true
 * when nonzero, kernels.rs:1305-1335). kind: 0 and, 1 or, 2 not. */
void orc_logical(int kind, const uint8_t *a, const uint8_t *b, uint8_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        out[i] = (uint8_t)(kind == 0 ? (a[i] != 0 && b[i] != 0) : kind == 1 ? (a[i] != 0 || b[i] != 0) : a[i] == 0);
}

/* [05-OP-53] where: the selected operand's stored bytes (NaN payloads and
 * signed zeros kept), kernels.rs:1338-1346. */
void orc_where(const uint8_t *cond, const void *a, const void *b, void *out, int64_t width, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        memcpy((char *)out + i * width, (const char *)(cond[i] ? a : b) + i * width, (size_t)width);
}

/* [05-OP-40] extrema cotangent (RiscOp::ExtremaAdjoint, crates/chelis-backend-
 * hip/src/kernels.rs:1030-1134): g where `right` (0: the left operand, 1:
 * the right) was selected by max (is_min 0) or min of (a, b), +0 elsewhere;
 * the left operand is selected when it is NaN, or when the right one is not
 * NaN and left >= right (min: <=). Float dtypes (bf16 / f16 compare decoded
 * values); the cotangent's stored bytes are copied. */
void orc_extrema_adjoint(int is_min, int right, int dt, const void *a, const void *b, const void *g, void *out,
                         int64_t n) {
    const int w = odt_width(dt);
    for (int64_t i = 0; i < n; ++i) {
        const double x = odt_float_at(dt, a, i), y = odt_float_at(dt, b, i);
        const int left = isnan(x) || (!isnan(y) && (is_min ? x <= y : x >= y));
        if (left != right) memcpy((char *)out + i * w, (const char *)g + i * w, (size_t)w);
        else memset((char *)out + i * w, 0, (size_t)w);
    }
}

/* Round-half-even right shift of a magnitude (the C lane's
 * chelis_host_round_shift_even_u64, crates/chelis-backend-c/src/
 * host_emit.rs:1705-1713). */
static uint64_t orc_rshift_even(uint64_t v, int s) {
    if (s <= 0) return v;
    if (s >= 64) return 0;
    const uint64_t q = v >> s, r = v & ((1ull << s) - 1ull), h = 1ull << (s - 1);
    return (r > h || (r == h && (q & 1ull))) ? q + 1 : q;
}
/* Pack sign, unbiased exponent of the leading bit and an (M+1)-bit rounded
 * significand into a 16-bit IEEE layout, carrying a round-up past M+1 bits
 * into the exponent and overflowing to infinity. */
static uint16_t orc_pack16(uint16_t sign, int e, uint64_t rounded, int E, int M) {
    const int bias = (1 << (E - 1)) - 1, emax = bias;
    if (rounded == (1ull << (M + 1))) {
        rounded >>= 1;
        ++e;
    }
    if (e > emax) return (uint16_t)(sign | ((uint32_t)((1 << E) - 1) << M));
    return (uint16_t)(sign | ((uint32_t)(e + bias) << M) | (uint32_t)(rounded & ((1ull << M) - 1ull)));
}
/* binary64 -> 16-bit IEEE (E exponent bits, M fraction bits) with one
 * rounding to nearest even; NaN to the canonical quiet NaN
 * (host_emit.rs:1715-1755). */
static uint16_t orc_f64_to_ieee16(double v, int E, int M) {
    uint64_t bits;
    memcpy(&bits, &v, 8);
    const uint16_t sign = (uint16_t)((bits >> 48) & 0x8000u);
    const int se = (int)((bits >> 52) & 0x7ff);
    const uint64_t man = bits & 0xfffffffffffffull;
    const int bias = (1 << (E - 1)) - 1;
    if (se == 0x7ff)
        return man ? (uint16_t)(((uint32_t)((1 << E) - 1) << M) | (1u << (M - 1)))
                   : (uint16_t)(sign | ((uint32_t)((1 << E) - 1) << M));
    if (se == 0 && man == 0) return sign;
    const int e = se ? se - 1023 : -1022;
    const uint64_t sig = se ? (man | (1ull << 52)) : man;
    if (se && e > bias) return (uint16_t)(sign | ((uint32_t)((1 << E) - 1) << M));
    if (se && e >= 1 - bias) return orc_pack16(sign, e, orc_rshift_even(sig, 52 - M), E, M);
    /* below the normal range: quantum 2^(1 - bias - M); a carry into the
     * leading bit position lands on the smallest normal's encoding */
    const int shift = (52 - M) + ((1 - bias) - e);
    return (uint16_t)(sign | (uint16_t)orc_rshift_even(sig, shift));
}
/* exact integer -> 16-bit IEEE with one rounding (host_emit.rs:1757-1776). */
static uint16_t orc_i64_to_ieee16(int64_t v, int E, int M) {
    const uint16_t sign = v < 0 ? 0x8000u : 0u;
    const uint64_t mag = v < 0 ? (uint64_t)(-(v + 1)) + 1ull : (uint64_t)v;
    if (!mag) return sign;
    int e = 63 - __builtin_clzll(mag);
    const int bias = (1 << (E - 1)) - 1;
    if (e > bias) return (uint16_t)(sign | ((uint32_t)((1 << E) - 1) << M));
    const uint64_t r = e > M ? orc_rshift_even(mag, e - M) : mag << (M - e);
    return orc_pack16(sign, e, r, E, M);
}

/* [04-NUM-14] checked cast, as the C lane's plan kinds
 * (crates/chelis-backend-c/src/host_emit.rs:1959-2120) and the runtime's
 * checks (crates/chelis-runtime/include/chelis_runtime.h:209-273):
 * identity for equal dtypes (stored bits kept); a float source to an
 * integer target traps domain unless finite and integral, then overflow
 * outside the target range; an integer or bool source to an integer target
 * traps overflow outside it; to bool, anything but 0 / 1 traps domain; to a
 * float target, one rounding to nearest even (NaN canonical). */
int64_t orc_cast(int src, int dst, const void *x, void *y, int64_t n, int32_t *kind) {
    int64_t first = -1;
    *kind = 0;
    const int ws = odt_width(src), wd = odt_width(dst);
    for (int64_t i = 0; i < n; ++i) {
        int fail = 0;
        if (src == dst) {
            memcpy((char *)y + i * wd, (const char *)x + i * ws, (size_t)wd);
            continue;
        }
        if (odt_is_float(src)) {
            const double v = odt_float_at(src, x, i);
            if (odt_is_float(dst)) {
                if (dst == ODT_F64) {
                    ((double *)y)[i] = nan64(v);
                } else if (dst == ODT_F32) {
                    ((float *)y)[i] = nan32((float)v);
                } else {
                    ((uint16_t *)y)[i] = dst == ODT_BF16 ? orc_f64_to_ieee16(v, 8, 7) : orc_f64_to_ieee16(v, 5, 10);
                }
            } else if (dst == ODT_BOOL) {
                if (!isfinite(v) || (v != 0.0 && v != 1.0)) fail = OFAIL_DOMAIN;
                ((uint8_t *)y)[i] = fail ? 0 : (uint8_t)(v == 1.0);
            } else {
                int64_t lo, hi;
                odt_limits(dst, &lo, &hi);
                if (!isfinite(v) || trunc(v) != v) fail = OFAIL_DOMAIN;
                else if (dst == ODT_I64 ? (v < -9223372036854775808.0 || v >= 9223372036854775808.0)
                                        : (v < (double)lo || v > (double)hi))
                    fail = OFAIL_OVERFLOW;
                odt_int_store(dst, y, i, fail ? 0 : (int64_t)v);
            }
        } else {
            const int64_t v = odt_int_at(src, x, i);
            if (dst == ODT_F64) {
                ((double *)y)[i] = (double)v;
            } else if (dst == ODT_F32) {
                ((float *)y)[i] = (float)v;
            } else if (dst == ODT_BF16 || dst == ODT_F16) {
                ((uint16_t *)y)[i] = dst == ODT_BF16 ? orc_i64_to_ieee16(v, 8, 7) : orc_i64_to_ieee16(v, 5, 10);
            } else if (dst == ODT_BOOL) {
                if (v != 0 && v != 1) fail = OFAIL_DOMAIN;
                ((uint8_t *)y)[i] = fail ? 0 : (uint8_t)(v == 1);
            } else {
                int64_t lo, hi;
                odt_limits(dst, &lo, &hi);
                if (v < lo || v > hi) fail = OFAIL_OVERFLOW;
                odt_int_store(dst, y, i, fail ? 0 : v);
            }
        }
        if (fail && first < 0) {
            first = i;
            *kind = fail;
        }
    }
    return first;
}

/* Checked signed-integer arithmetic at the operand width
 * (crates/chelis-numeric-core/src/dtype_semantics.rs:930-985 binary,
 * :1015-1030 unary): add, sub, mul overflow outside the width's range;
 * floor_div / trunc_div / mod trap division by zero on a zero divisor,
 * floor_div and trunc_div overflow on MIN / -1 (mod of -1 is 0); floor_div
 * rounds the truncated quotient down when the remainder's sign differs from
 * the divisor's; max_elem / min_elem never trap. op: 0 add, 1 sub, 2 mul,
 * 3 floor_div, 4 trunc_div, 5 mod, 6 max_elem, 7 min_elem; the bitwise ops
 * of [05-OP-47] (crates/chelis-backend-c/src/emit.rs:2354-2362): 8 bitand,
 * 9 bitor, 10 bitxor on the two's-complement bits, 11 shl, 12 shr. */
int64_t orc_int_binary(int op, int dt, const void *a, const void *b, void *y, int64_t n, int32_t *kind) {
    int64_t first = -1, lo, hi;
    *kind = 0;
    odt_limits(dt, &lo, &hi);
    for (int64_t i = 0; i < n; ++i) {
        const int64_t x = odt_int_at(dt, a, i), z = odt_int_at(dt, b, i);
        int64_t r = 0;
        int fail = 0;
        switch (op) {
            case 0: fail = (__builtin_add_overflow(x, z, &r) || r < lo || r > hi) ? OFAIL_OVERFLOW : 0; break;
            case 1: fail = (__builtin_sub_overflow(x, z, &r) || r < lo || r > hi) ? OFAIL_OVERFLOW : 0; break;
            case 2: fail = (__builtin_mul_overflow(x, z, &r) || r < lo || r > hi) ? OFAIL_OVERFLOW : 0; break;
            case 3: case 4: case 5:
                if (z == 0) {
                    fail = OFAIL_DIVZERO;
                } else if (op == 5) {
                    r = z == -1 ? 0 : x % z;
                } else if (x == lo && z == -1) {
                    fail = OFAIL_OVERFLOW;
                } else {
                    r = x / z;
                    if (op == 3 && x % z != 0 && ((x % z < 0) != (z < 0))) r -= 1;
                }
                break;
            case 6: r = x > z ? x : z; break;
            case 7: r = x < z ? x : z; break;
            case 8: r = x & z; break;
            case 9: r = x | z; break;
            case 10: r = x ^ z; break;
            default: {
                /* [04-NUM-13] shifts (crates/chelis-runtime/include/
                 * chelis_runtime.h:297-330): the w-bit pattern moved as an
                 * unsigned word, read back as two's complement; a count of w
                 * or more gives 0 (shr of a negative value: -1); a negative
                 * count fails (the C lane's "shift amount must be
                 * non-negative" trap, here domain) */
                const int w = odt_bits(dt);
                const uint64_t mask = w == 64 ? ~0ull : ((1ull << w) - 1);
                const uint64_t raw = (uint64_t)x & mask;
                uint64_t v;
                if (z < 0) {
                    fail = OFAIL_DOMAIN;
                    v = 0;
                } else if (op == 11) {
                    v = z >= w ? 0 : (raw << z) & mask;
                } else {
                    const int neg = (raw >> (w - 1)) & 1;
                    if (z >= w) v = neg ? mask : 0;
                    else {
                        v = raw >> z;
                        if (neg && z > 0) v |= mask & ~(mask >> z);
                    }
                }
                r = (v >> (w - 1)) & 1 ? (int64_t)(v | ~mask) : (int64_t)v;
                break;
            }
        }
        odt_int_store(dt, y, i, fail ? 0 : r);
        if (fail && first < 0) {
            first = i;
            *kind = fail;
        }
    }
    return first;
}
/* op: 0 neg, 1 abs; both overflow on the width's minimum. */
int64_t orc_int_unary(int op, int dt, const void *x, void *y, int64_t n, int32_t *kind) {
    int64_t first = -1, lo, hi;
    *kind = 0;
    odt_limits(dt, &lo, &hi);
    for (int64_t i = 0; i < n; ++i) {
        const int64_t v = odt_int_at(dt, x, i);
        const int fail = v == lo ? OFAIL_OVERFLOW : 0;
        odt_int_store(dt, y, i, fail ? 0 : (op == 0 || v < 0) ? -v : v);
        if (fail && first < 0) {
            first = i;
            *kind = fail;
        }
    }
    return first;
}

/* Gather (RiscOp::Gather{axis, batch_rank}, crates/chelis-dag-core/src/
 * dag.rs:1349-1356) with the HIP lane's geometry (emit.rs:3807-3842,
 * kernels.rs:2557-2597): values viewed as [before, axis_size, after], the
 * result as [before, index_count, after] where index_count counts the
 * indices past their batch_rank leading axes, which pair with the values'
 * leading axes; result element (b, j, d) reads values (b, g, d) with g the
 * index at (batch of b, j). An index outside [0, axis_size) traps domain;
 * its element is zero. Values elements are `width` bytes; indices i32
 * (idx_dt 2) or i64 (idx_dt 4), contiguous. */
int64_t orc_gather(const void *values, int64_t width, int64_t before, int64_t axis_size, int64_t after,
                   const void *idx, int idx_dt, int64_t index_count, int64_t batch_count, void *out, int32_t *kind) {
    int64_t first = -1;
    *kind = 0;
    const int64_t outer_per_batch = (batch_count == 0 || before == 0) ? 1 : before / batch_count;
    const int64_t total = before * index_count * after;
    for (int64_t i = 0; i < total; ++i) {
        const int64_t d = i % after, t = i / after, j = t % index_count, b = t / index_count;
        const int64_t pos = (b / outer_per_batch) * index_count + j;
        const int64_t g = odt_int_at(idx_dt, idx, pos);
        char *dst = (char *)out + i * width;
        if (g < 0 || g >= axis_size) {
            memset(dst, 0, (size_t)width);
            if (first < 0) {
                first = i;
                *kind = OFAIL_DOMAIN;
            }
            continue;
        }
        memcpy(dst, (const char *)values + ((b * axis_size + g) * after + d) * width, (size_t)width);
    }
    return first;
}

/* [05-OP-33] ordered inclusive scan along the middle axis of a contiguous
 * [outer, n, inner] tensor: the C lane's chelis_tensor_cumsum
 * (crates/chelis-runtime/src/lib.rs:7020-7105). Per line, in the order
 * outer, inner, step: the first leaf is the first prefix (NaN canonical),
 * each later prefix is the previous one plus the leaf at the accumulator
 * width - binary32 for bf16 / f16, i32 for i8 / i16, the dtype otherwise -
 * and each prefix is stored at the result dtype (bf16 / f16 rounded from the
 * binary32 prefix; i8 / i16 scan into i32). reverse scans each line from its
 * end (the decreasing direction, crates/chelis-backend-c/src/emit.rs:
 * 8000-8075). An integer prefix outside the accumulator's range fails
 * overflow; the return is that prefix's position in the evaluation order
 * ((o * inner + j) * n + step), or -1. */
int64_t orc_cumsum(int dt, const void *x, void *y, int64_t outer, int64_t n, int64_t inner, int reverse,
                   int32_t *kind) {
    int64_t first = -1;
    *kind = 0;
    const int idt = (dt == ODT_I8 || dt == ODT_I16) ? ODT_I32 : dt;  /* result dtype */
    int64_t lo, hi;
    odt_limits(idt == ODT_I64 ? ODT_I64 : ODT_I32, &lo, &hi);
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t j = 0; j < inner; ++j) {
            double facc = 0.0;
            float sacc = 0.0f;
            int64_t iacc = 0;
            for (int64_t step = 0; step < n; ++step) {
                const int64_t pos = reverse ? n - 1 - step : step;
                const int64_t f = (o * n + pos) * inner + j;
                if (dt == ODT_F64) {
                    const double v = ((const double *)x)[f];
                    facc = nan64(step == 0 ? v : facc + v);
                    ((double *)y)[f] = facc;
                } else if (odt_is_float(dt)) {
                    const float v = (float)odt_float_at(dt, x, f);
                    sacc = nan32(step == 0 ? v : sacc + v);
                    if (dt == ODT_F32) ((float *)y)[f] = sacc;
                    else ((uint16_t *)y)[f] = orc_enc16(dt == ODT_BF16 ? 0 : 1, sacc);
                } else {
                    const int64_t v = odt_int_at(dt, x, f);
                    int64_t r = v;
                    int fail = 0;
                    if (step > 0) fail = __builtin_add_overflow(iacc, v, &r) || r < lo || r > hi;
                    if (fail && first < 0) {
                        first = (o * inner + j) * n + step;
                        *kind = OFAIL_OVERFLOW;
                    }
                    iacc = fail ? 0 : r;
                    odt_int_store(idt, y, f, iacc);
                }
            }
        }
    return first;
}

/* Movement with bounds over contiguous row-major arrays of `width`-byte
 * elements (rank <= 8).
 * Pad (RiscOp::Pad{padding, fill}): the C lane fills the result with the
 * fill's bits, then copies source element i to the result at its
 * coordinates plus `lo` (crates/chelis-backend-c/src/emit.rs:10880-10954).
 * Shrink / Stride (emit.rs:10956-11042): result element o reads the source
 * at o * step + start on every axis (shrink: step 1; stride: start 0). */
static void orc_coords(int64_t i, int rank, const int64_t *shape, int64_t *c) {
    for (int a = rank - 1; a >= 0; --a) {
        c[a] = shape[a] ? i % shape[a] : 0;
        i = shape[a] ? i / shape[a] : 0;
    }
}
static int64_t orc_flat(int rank, const int64_t *shape, const int64_t *c) {
    int64_t f = 0;
    for (int a = 0; a < rank; ++a) f = f * shape[a] + c[a];
    return f;
}
void orc_pad(int width, const void *x, int rank, const int64_t *src_shape, const int64_t *lo,
             const int64_t *out_shape, uint64_t fill, void *y) {
    int64_t n_out = 1, n_src = 1, c[8];
    for (int a = 0; a < rank; ++a) {
        n_out *= out_shape[a];
        n_src *= src_shape[a];
    }
    for (int64_t i = 0; i < n_out; ++i) memcpy((char *)y + i * width, &fill, (size_t)width);
    for (int64_t i = 0; i < n_src; ++i) {
        orc_coords(i, rank, src_shape, c);
        for (int a = 0; a < rank; ++a) c[a] += lo[a];
        memcpy((char *)y + orc_flat(rank, out_shape, c) * width, (const char *)x + i * width, (size_t)width);
    }
}
void orc_slice(int width, const void *x, int rank, const int64_t *src_shape, const int64_t *start,
               const int64_t *step, const int64_t *out_shape, void *y) {
    int64_t n_out = 1, c[8];
    for (int a = 0; a < rank; ++a) n_out *= out_shape[a];
    for (int64_t i = 0; i < n_out; ++i) {
        orc_coords(i, rank, out_shape, c);
        for (int a = 0; a < rank; ++a) c[a] = c[a] * step[a] + start[a];
        memcpy((char *)y + i * width, (const char *)x + orc_flat(rank, src_shape, c) * width, (size_t)width);
    }
}

/* Sparse scatters (RiscOp::ScatterAdd / Scatter / ScatterElements,
 * crates/chelis-dag-core/src/dag.rs:1360-1404) as the C lane runs them
 * (crates/chelis-backend-c/src/emit.rs:7382-7470): the result starts as the
 * target; the updates are visited in ascending row-major position, each
 * index checked against the axis extent (the first outside it fails
 * domain: its position is returned). `dest` holds each update's flat
 * destination in the row-major target. Replace (add = 0) stores each update
 * in turn, so the last write wins. Add records the destinations, orders
 * them by a stable counting sort, and folds per destination - its target
 * value, then its updates in ascending position - level by level, adjacent
 * pairs left to right, an odd tail carried up (emit.rs:7772-7801,
 * 7842-7990): floats add at the dtype (bf16 / f16 in binary32, rounded at
 * every node), the total NaN-canonical; integers fail overflow at the first
 * node outside the width (returned as n + the destination). */
static int64_t orc_scatter_apply(int add, int dt, const int64_t *dest, int64_t n, const void *upd, void *out,
                                 int64_t out_n, int32_t *kind) {
    const int w = odt_width(dt);
    if (!add) {
        for (int64_t i = 0; i < n; ++i) memcpy((char *)out + dest[i] * w, (const char *)upd + i * w, (size_t)w);
        return -1;
    }
    int64_t *end = (int64_t *)calloc((size_t)(out_n + 1), sizeof(int64_t));
    int64_t *order = (int64_t *)malloc((size_t)(n + 1) * sizeof(int64_t));
    double *lv = (double *)malloc((size_t)(n + 2) * sizeof(double));
    int64_t *li = (int64_t *)malloc((size_t)(n + 2) * sizeof(int64_t));
    int64_t first = -1, lo, hi;
    odt_limits(dt, &lo, &hi);
    for (int64_t i = 0; i < n; ++i) end[dest[i]] += 1;
    for (int64_t d = 1; d < out_n; ++d) end[d] += end[d - 1];
    for (int64_t i = n - 1; i >= 0; --i) order[--end[dest[i]]] = i;
    for (int64_t d = 0; d < out_n && first < 0; ++d) {
        const int64_t a = end[d], b = d + 1 < out_n ? end[d + 1] : n;
        if (a == b) continue;
        int64_t leaves = b - a + 1;
        if (odt_is_float(dt)) {
            lv[0] = odt_float_at(dt, out, d);
            for (int64_t k = a; k < b; ++k) lv[k - a + 1] = odt_float_at(dt, upd, order[k]);
        } else {
            li[0] = odt_int_at(dt, out, d);
            for (int64_t k = a; k < b; ++k) li[k - a + 1] = odt_int_at(dt, upd, order[k]);
        }
        while (leaves > 1 && first < 0) {
            const int64_t next = leaves / 2 + leaves % 2;
            for (int64_t q = 0; q < next; ++q) {
                const int64_t l = 2 * q, r = l + 1;
                if (r >= leaves) {
                    lv[q] = lv[l];
                    li[q] = li[l];
                    continue;
                }
                switch (dt) {
                    case ODT_F32: lv[q] = (double)((float)lv[l] + (float)lv[r]); break;
                    case ODT_F64: lv[q] = lv[l] + lv[r]; break;
                    case ODT_BF16: case ODT_F16: {
                        const int k16 = dt == ODT_BF16 ? 0 : 1;
                        lv[q] = (double)orc_dec16(k16, orc_enc16(k16, (float)lv[l] + (float)lv[r]));
                        break;
                    }
                    default: {
                        /* operands within the width: only i64 can leave int64 */
                        int64_t t64 = 0;
                        const int bad = __builtin_add_overflow(li[l], li[r], &t64);
                        if (bad || t64 < lo || t64 > hi) {
                            first = n + d;
                            *kind = OFAIL_OVERFLOW;
                        }
                        li[q] = t64;
                    }
                }
            }
            leaves = next;
        }
        if (first >= 0) break;
        switch (dt) {
            case ODT_F32: ((float *)out)[d] = nan32((float)lv[0]); break;
            case ODT_F64: ((double *)out)[d] = nan64(lv[0]); break;
            case ODT_BF16: ((uint16_t *)out)[d] = orc_enc16(0, (float)lv[0]); break;
            case ODT_F16: ((uint16_t *)out)[d] = orc_enc16(1, (float)lv[0]); break;
            default: odt_int_store(dt, out, d, li[0]);
        }
    }
    free(end);
    free(order);
    free(lv);
    free(li);
    return first;
}
/* Scatter / ScatterAdd (hyperplane form, the gather's geometry above):
 * update (b, j, d) of [before, index_count, after] goes to the target at
 * (b, idx[batch of b, j], d) of [before, axis_size, after]. */
int64_t orc_scatter(int add, int dt, const void *target, const int64_t *idx, const void *upd, void *out,
                    int64_t before, int64_t axis_size, int64_t after, int64_t index_count, int64_t outer_per_batch,
                    int32_t *kind) {
    const int w = odt_width(dt);
    const int64_t out_n = before * axis_size * after, n = before * index_count * after;
    *kind = 0;
    memcpy(out, target, (size_t)(out_n * w));
    int64_t *dest = (int64_t *)malloc((size_t)(n + 1) * sizeof(int64_t));
    for (int64_t i = 0; i < n; ++i) {
        const int64_t d = i % after, t = i / after, j = t % index_count, b = t / index_count;
        const int64_t g = idx[(b / outer_per_batch) * index_count + j];
        if (g < 0 || g >= axis_size) {
            free(dest);
            *kind = OFAIL_DOMAIN;
            return i;
        }
        dest[i] = (b * axis_size + g) * after + d;
    }
    const int64_t r = orc_scatter_apply(add, dt, dest, n, upd, out, out_n, kind);
    free(dest);
    return r;
}
/* ScatterElements (dag.rs:1386-1404): the update at coordinates c of the
 * indices' shape goes to the target at c with c[axis] = idx[c]. */
int64_t orc_scatter_elements(int dt, const void *target, const int64_t *idx, const void *upd, void *out, int rank,
                             const int64_t *idx_shape, const int64_t *target_shape, int axis, int32_t *kind) {
    const int w = odt_width(dt);
    int64_t out_n = 1, n = 1, c[8];
    for (int a = 0; a < rank; ++a) {
        out_n *= target_shape[a];
        n *= idx_shape[a];
    }
    *kind = 0;
    memcpy(out, target, (size_t)(out_n * w));
    int64_t *dest = (int64_t *)malloc((size_t)(n + 1) * sizeof(int64_t));
    for (int64_t i = 0; i < n; ++i) {
        orc_coords(i, rank, idx_shape, c);
        if (idx[i] < 0 || idx[i] >= target_shape[axis]) {
            free(dest);
            *kind = OFAIL_DOMAIN;
            return i;
        }
        c[axis] = idx[i];
        dest[i] = orc_flat(rank, target_shape, c);
    }
    const int64_t r = orc_scatter_apply(0, dt, dest, n, upd, out, out_n, kind);
    free(dest);
    return r;
}

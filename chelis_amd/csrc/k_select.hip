// Comparison, logical, where, checked casts, checked integer arithmetic and
// gather on gfx950: the node kinds the reference HIP lane launches one
// kernel each for beside its float chains (crates/chelis-backend-hip/src/
// kernels.rs:1270-1346 comparison / logical / where, :1382 and
// emit.rs:2413 casts, kernels.rs:769-866 and :1434 the trapping integer
// kernels, :2557-2597 gather). Where the two reference lanes differ the C
// lane's semantics hold: integer add and mul are checked as sub and abs are
// (crates/chelis-numeric-core/src/dtype_semantics.rs:930-1030), and a cast
// is [04-NUM-14]'s checked cast with the C lane's single roundings
// (crates/chelis-backend-c/src/host_emit.rs:1700-2120).
//
// Every map is a grid-stride loop over the output's elements, one per lane
// per step (coalesced), over operands collapsed to at most four strided
// axes (stride 0 broadcasts). A failing element ([04-NUM-9]) stores zero
// and contributes a record key: bits 63..42 the launch's sequence number,
// 41..2 the element's row-major index, 1..0 the kind. The wave joins its
// keys and one lane merges them into the device's record word with an
// atomic max of the complement, so the word keeps the lowest key - the
// earliest launch's lowest-index offender, [04-NUM-15] - and 0 means none.
#include <algorithm>
#include <limits>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include <hipcub/hipcub.hpp>

#include "hip_common.h"
#include "narrow.h"
#include "strided.h"

namespace chelis {
namespace {

enum : int { kOverflow = 1, kDomain = 2, kDivZero = 3 };

// ---------------------------------------------------------------- element types
template <int DT> struct Dt;
template <> struct Dt<CHELIS_DTYPE_F32> { using S = float; static constexpr bool kFloat = true; };
template <> struct Dt<CHELIS_DTYPE_F64> { using S = double; static constexpr bool kFloat = true; };
template <> struct Dt<CHELIS_DTYPE_BF16> { using S = uint16_t; static constexpr bool kFloat = true; };
template <> struct Dt<CHELIS_DTYPE_F16> { using S = uint16_t; static constexpr bool kFloat = true; };
template <> struct Dt<CHELIS_DTYPE_I8> { using S = int8_t; static constexpr bool kFloat = false; };
template <> struct Dt<CHELIS_DTYPE_I16> { using S = int16_t; static constexpr bool kFloat = false; };
template <> struct Dt<CHELIS_DTYPE_I32> { using S = int32_t; static constexpr bool kFloat = false; };
template <> struct Dt<CHELIS_DTYPE_I64> { using S = int64_t; static constexpr bool kFloat = false; };
template <> struct Dt<CHELIS_DTYPE_BOOL> { using S = uint8_t; static constexpr bool kFloat = false; };

// The value a comparison sees: bf16 / f16 decoded to binary32 (exact),
// every other dtype its stored value (kernels.rs:1266-1268).
template <int DT>
__device__ inline auto semantic(typename Dt<DT>::S v) {
    if constexpr (DT == CHELIS_DTYPE_BF16) return bf16_to_f32(v);
    else if constexpr (DT == CHELIS_DTYPE_F16) return f16_to_f32(v);
    else return v;
}
// A float element's exact value in binary64.
template <int DT>
__device__ inline double widen(typename Dt<DT>::S v) {
    return (double)semantic<DT>(v);
}

// ---------------------------------------------------------------- operands
struct Ops {
    const void *p[3];
    int64_t st[3][kMaxRank];
};

template <int N>
__device__ inline void offsets(const Ops &o, const Shape &sh, int64_t idx, int64_t (&off)[N]) {
    if (sh.rank <= 1) {
#pragma unroll
        for (int k = 0; k < N; ++k) off[k] = idx * o.st[k][0];
        return;
    }
    int64_t coord[kMaxRank];
    int64_t rem = idx;
#pragma unroll
    for (int a = kMaxRank - 1; a >= 0; --a) {
        if (a < sh.rank) {
            coord[a] = rem % sh.ext[a];
            rem /= sh.ext[a];
        } else {
            coord[a] = 0;
        }
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
        int64_t s = 0;
#pragma unroll
        for (int a = 0; a < kMaxRank; ++a) s += coord[a] * o.st[k][a];
        off[k] = s;
    }
}

// A record key: ~(launch sequence << kSeqShift | element index << 2 | kind),
// so the atomic maximum keeps the earliest launch's lowest failing element.
constexpr int kSeqShift = 42;

__device__ inline unsigned long long fail_key(uint64_t seq, int64_t i, int kind) {
    return ~(seq | ((uint64_t)i << 2) | (uint64_t)kind);
}

// Joins the wave's failure keys (0: none) and merges the largest into the
// record word from one lane. Every lane of the wave calls it in the same
// loop step (the loop bound is uniform).
__device__ inline void merge_failures(unsigned long long k, unsigned long long *rec) {
    if (!__any(k != 0ull)) return;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const unsigned long long o = __shfl_xor(k, m);
        k = o > k ? o : k;
    }
    if ((threadIdx.x & 63) == 0) atomicMax(rec, k);
}

// The kernels below that index by thread run 256 threads per workgroup
// (their launches pass that count): the constant, not blockDim.x, which
// is a vector load from the dispatch packet at the start of each wave.
constexpr int kSelectThreads = 256;

// One element per lane per step; the block's steps start at a uniform base
// so a wave's lanes are always in the same step (lanes past the end take no
// element and report no failure).
template <class F>
__global__ __launch_bounds__(256) void map_kernel(F f, Ops o, Shape sh, int64_t count, unsigned long long *rec) {
    const int64_t stride = (int64_t)gridDim.x * kSelectThreads;
    for (int64_t base = (int64_t)blockIdx.x * kSelectThreads; base < count; base += stride) {
        const int64_t i = base + threadIdx.x;
        unsigned long long k = 0ull;
        if (i < count) {
            int64_t off[F::N];
            offsets(o, sh, i, off);
            k = f(i, o, off);
        }
        if constexpr (F::kTraps) merge_failures(k, rec);
    }
}

// ---------------------------------------------------------------- comparison, logical, where
template <typename V>
__device__ inline bool compare_values(int kind, V x, V y) {
    switch (kind) {
        case CHELIS_CMP_CMPLT: case CHELIS_CMP_LT: return x < y;
        case CHELIS_CMP_EQ: return x == y;
        case CHELIS_CMP_NEQ: return x != y;
        case CHELIS_CMP_GT: return x > y;
        case CHELIS_CMP_GTE: return x >= y;
        default: return x <= y;
    }
}

template <int DT>
struct CompareOp {
    static constexpr int N = 2;
    static constexpr bool kTraps = false;
    int32_t kind;
    uint8_t *out;
    __device__ unsigned long long operator()(int64_t i, const Ops &o, const int64_t (&off)[2]) const {
        using S = typename Dt<DT>::S;
        const auto x = semantic<DT>(static_cast<const S *>(o.p[0])[off[0]]);
        const auto y = semantic<DT>(static_cast<const S *>(o.p[1])[off[1]]);
        out[i] = (uint8_t)compare_values(kind, x, y);
        return 0ull;
    }
};

// A Bool8 byte is true when nonzero (kernels.rs:1305-1335).
struct LogicalOp {
    static constexpr int N = 2;
    static constexpr bool kTraps = false;
    int32_t kind;
    uint8_t *out;
    __device__ unsigned long long operator()(int64_t i, const Ops &o, const int64_t (&off)[2]) const {
        const uint8_t a = static_cast<const uint8_t *>(o.p[0])[off[0]];
        const uint8_t b = static_cast<const uint8_t *>(o.p[1])[off[1]];
        out[i] = (uint8_t)(kind == CHELIS_LOGICAL_AND ? (a != 0 && b != 0)
                           : kind == CHELIS_LOGICAL_OR ? (a != 0 || b != 0) : a == 0);
        return 0ull;
    }
};

// [05-OP-53]: the selected operand's stored bits; the other is not read.
template <typename U>
struct WhereOp {
    static constexpr int N = 3;
    static constexpr bool kTraps = false;
    U *out;
    __device__ unsigned long long operator()(int64_t i, const Ops &o, const int64_t (&off)[3]) const {
        const bool c = static_cast<const uint8_t *>(o.p[0])[off[0]] != 0;
        out[i] = c ? static_cast<const U *>(o.p[1])[off[1]] : static_cast<const U *>(o.p[2])[off[2]];
        return 0ull;
    }
};

// [05-OP-40] extrema cotangent (kernels.rs:1030-1134): the cotangent where
// `operand` was selected, +0 elsewhere. max selects the left operand when it
// is NaN, or when the right one is not NaN and left >= right (min: <=), the
// first-operand tie rule of max_elem / min_elem; bf16 / f16 compare decoded
// values and pass the cotangent's stored bits.
template <int DT>
struct ExtremaAdjointOp {
    static constexpr int N = 3;
    static constexpr bool kTraps = false;
    int32_t is_min, right;
    typename Dt<DT>::S *out;
    __device__ unsigned long long operator()(int64_t i, const Ops &o, const int64_t (&off)[3]) const {
        using S = typename Dt<DT>::S;
        const auto a = semantic<DT>(static_cast<const S *>(o.p[0])[off[0]]);
        const auto b = semantic<DT>(static_cast<const S *>(o.p[1])[off[1]]);
        const bool left = a != a || (b == b && (is_min ? a <= b : a >= b));
        out[i] = left != (right != 0) ? static_cast<const S *>(o.p[2])[off[2]] : S{};
        return 0ull;
    }
};

// ---------------------------------------------------------------- checked cast
// Round-half-even right shift of a magnitude.
__device__ inline uint64_t rshift_even(uint64_t v, int s) {
    if (s <= 0) return v;
    if (s >= 64) return 0;
    const uint64_t q = v >> s, r = v & ((1ull << s) - 1ull), h = 1ull << (s - 1);
    return (r > h || (r == h && (q & 1ull))) ? q + 1 : q;
}
// Sign, unbiased exponent of the leading bit and an (M+1)-bit rounded
// significand packed into an IEEE layout with E exponent bits; a round-up
// past M+1 bits carries into the exponent, overflow gives infinity.
template <int E, int M, typename U>
__device__ inline U pack_ieee(U sign, int e, uint64_t rounded) {
    constexpr int bias = (1 << (E - 1)) - 1;
    if (rounded == (1ull << (M + 1))) {
        rounded >>= 1;
        ++e;
    }
    if (e > bias) return (U)(sign | ((U)((1 << E) - 1) << M));
    return (U)(sign | ((U)(e + bias) << M) | (U)(rounded & ((1ull << M) - 1ull)));
}
// An exact integer to an IEEE format with one rounding to nearest even.
template <int E, int M, typename U>
__device__ inline U int_to_ieee(int64_t v) {
    const U sign = v < 0 ? (U)((U)1 << (E + M)) : (U)0;
    const uint64_t mag = v < 0 ? (uint64_t)(-(v + 1)) + 1ull : (uint64_t)v;
    if (!mag) return sign;
    const int e = 63 - __builtin_clzll(mag);
    constexpr int bias = (1 << (E - 1)) - 1;
    if (e > bias) return (U)(sign | ((U)((1 << E) - 1) << M));
    const uint64_t r = e > M ? rshift_even(mag, e - M) : mag << (M - e);
    return pack_ieee<E, M, U>(sign, e, r);
}
// binary64 to a 16-bit IEEE format with one rounding to nearest even; NaN
// to the format's canonical quiet NaN (host_emit.rs:1715-1755).
template <int E, int M>
__device__ inline uint16_t f64_to_ieee16(double v) {
    const uint64_t bits = __builtin_bit_cast(uint64_t, v);
    const uint16_t sign = (uint16_t)((bits >> 48) & 0x8000u);
    const int se = (int)((bits >> 52) & 0x7ff);
    const uint64_t man = bits & 0xfffffffffffffull;
    constexpr int bias = (1 << (E - 1)) - 1;
    constexpr uint16_t inf = (uint16_t)(((1 << E) - 1) << M);
    if (se == 0x7ff) return man ? (uint16_t)(inf | (1u << (M - 1))) : (uint16_t)(sign | inf);
    if (se == 0 && man == 0) return sign;
    const int e = se ? se - 1023 : -1022;
    const uint64_t sig = se ? (man | (1ull << 52)) : man;
    if (se && e > bias) return (uint16_t)(sign | inf);
    if (se && e >= 1 - bias) return pack_ieee<E, M, uint16_t>(sign, e, rshift_even(sig, 52 - M));
    // below the normal range: quantum 2^(1 - bias - M); a carry into the
    // leading position is the smallest normal's encoding
    return (uint16_t)(sign | (uint16_t)rshift_even(sig, (52 - M) + ((1 - bias) - e)));
}

template <int DT> constexpr int64_t int_min() {
    return DT == CHELIS_DTYPE_I8 ? -128 : DT == CHELIS_DTYPE_I16 ? -32768 : DT == CHELIS_DTYPE_I32 ? -2147483648LL
                                                                          : (-9223372036854775807LL - 1);
}
template <int DT> constexpr int64_t int_max() {
    return DT == CHELIS_DTYPE_I8 ? 127 : DT == CHELIS_DTYPE_I16 ? 32767 : DT == CHELIS_DTYPE_I32 ? 2147483647LL
                                                                        : 9223372036854775807LL;
}

// [04-NUM-14] for one element: the failure kind, or 0 with *r set.
template <int SRC, int DST>
__device__ inline int cast_one(typename Dt<SRC>::S v, typename Dt<DST>::S *r) {
    using D = typename Dt<DST>::S;
    if constexpr (SRC == DST) {
        *r = v;  // identity keeps the stored bits
    } else if constexpr (Dt<SRC>::kFloat) {
        const double x = widen<SRC>(v);
        if constexpr (DST == CHELIS_DTYPE_F64) {
            *r = x != x ? __builtin_bit_cast(double, 0x7ff8000000000000ull) : x;
        } else if constexpr (DST == CHELIS_DTYPE_F32) {
            const float f = (float)x;
            *r = f != f ? __builtin_bit_cast(float, 0x7fc00000u) : f;
        } else if constexpr (DST == CHELIS_DTYPE_BF16) {
            *r = f64_to_ieee16<8, 7>(x);
        } else if constexpr (DST == CHELIS_DTYPE_F16) {
            *r = f64_to_ieee16<5, 10>(x);
        } else if constexpr (DST == CHELIS_DTYPE_BOOL) {
            if (!__builtin_isfinite(x) || (x != 0.0 && x != 1.0)) return kDomain;
            *r = (D)(x == 1.0);
        } else {
            if (!__builtin_isfinite(x) || __builtin_trunc(x) != x) return kDomain;
            if (DST == CHELIS_DTYPE_I64 ? (x < -9223372036854775808.0 || x >= 9223372036854775808.0)
                                        : (x < (double)int_min<DST>() || x > (double)int_max<DST>()))
                return kOverflow;
            *r = (D)(int64_t)x;
        }
    } else {
        const int64_t x = (int64_t)v;
        if constexpr (DST == CHELIS_DTYPE_F64) {
            *r = __builtin_bit_cast(double, int_to_ieee<11, 52, uint64_t>(x));
        } else if constexpr (DST == CHELIS_DTYPE_F32) {
            *r = __builtin_bit_cast(float, int_to_ieee<8, 23, uint32_t>(x));
        } else if constexpr (DST == CHELIS_DTYPE_BF16) {
            *r = int_to_ieee<8, 7, uint16_t>(x);
        } else if constexpr (DST == CHELIS_DTYPE_F16) {
            *r = int_to_ieee<5, 10, uint16_t>(x);
        } else if constexpr (DST == CHELIS_DTYPE_BOOL) {
            if (x != 0 && x != 1) return kDomain;
            *r = (D)(x == 1);
        } else {
            if (x < int_min<DST>() || x > int_max<DST>()) return kOverflow;
            *r = (D)x;
        }
    }
    return 0;
}

template <int SRC, int DST>
struct CastOp {
    static constexpr int N = 1;
    static constexpr bool kTraps = true;
    typename Dt<DST>::S *out;
    uint64_t seq;
    __device__ unsigned long long operator()(int64_t i, const Ops &o, const int64_t (&off)[1]) const {
        using S = typename Dt<SRC>::S;
        using D = typename Dt<DST>::S;
        D r{};
        const int kind = cast_one<SRC, DST>(static_cast<const S *>(o.p[0])[off[0]], &r);
        out[i] = kind ? D{} : r;
        return kind ? fail_key(seq, i, kind) : 0ull;
    }
};

// ---------------------------------------------------------------- checked integer arithmetic
template <typename T>
__device__ inline int int_binary(int op, T x, T z, T *r) {
    constexpr T lo = std::numeric_limits<T>::min();
    switch (op) {
        case CHELIS_INT_ADD: return __builtin_add_overflow(x, z, r) ? kOverflow : 0;
        case CHELIS_INT_SUB: return __builtin_sub_overflow(x, z, r) ? kOverflow : 0;
        case CHELIS_INT_MUL: return __builtin_mul_overflow(x, z, r) ? kOverflow : 0;
        case CHELIS_INT_FLOOR_DIV: case CHELIS_INT_TRUNC_DIV: case CHELIS_INT_MOD: {
            if (z == 0) return kDivZero;
            if (op == CHELIS_INT_MOD) {
                *r = z == (T)-1 ? (T)0 : (T)(x % z);
                return 0;
            }
            if (x == lo && z == (T)-1) return kOverflow;
            T q = (T)(x / z);
            const T m = (T)(x % z);
            if (op == CHELIS_INT_FLOOR_DIV && m != 0 && ((m < 0) != (z < 0))) q = (T)(q - 1);
            *r = q;
            return 0;
        }
        case CHELIS_INT_MAX_ELEM: *r = x > z ? x : z; return 0;
        case CHELIS_INT_MIN_ELEM: *r = x < z ? x : z; return 0;
        case CHELIS_INT_BITAND: *r = (T)(x & z); return 0;
        case CHELIS_INT_BITOR: *r = (T)(x | z); return 0;
        case CHELIS_INT_BITXOR: *r = (T)(x ^ z); return 0;
        default: {
            // [04-NUM-13]: the bits move as the unsigned w-bit pattern; a
            // count of w or more empties it (shr: fills it with the sign)
            using U = std::make_unsigned_t<T>;
            constexpr int W = 8 * (int)sizeof(T);
            if (z < 0) return kDomain;
            const U u = (U)x;
            if (op == CHELIS_INT_SHL) {
                *r = z >= W ? (T)0 : (T)(U)(u << (int)z);
            } else {
                const bool neg = x < 0;
                if (z >= W) *r = neg ? (T)-1 : (T)0;
                else {
                    U v = (U)(u >> (int)z);
                    if (neg && z != 0) v = (U)(v | (U)~((U)~(U)0 >> (int)z));
                    *r = (T)v;
                }
            }
            return 0;
        }
    }
}

template <typename T>
struct IntBinaryOp {
    static constexpr int N = 2;
    static constexpr bool kTraps = true;
    int32_t op;
    T *out;
    uint64_t seq;
    __device__ unsigned long long operator()(int64_t i, const Ops &o, const int64_t (&off)[2]) const {
        T r = 0;
        const int kind = int_binary<T>(op, static_cast<const T *>(o.p[0])[off[0]],
                                       static_cast<const T *>(o.p[1])[off[1]], &r);
        out[i] = kind ? (T)0 : r;
        return kind ? fail_key(seq, i, kind) : 0ull;
    }
};

template <typename T>
struct IntUnaryOp {
    static constexpr int N = 1;
    static constexpr bool kTraps = true;
    int32_t op;
    T *out;
    uint64_t seq;
    __device__ unsigned long long operator()(int64_t i, const Ops &o, const int64_t (&off)[1]) const {
        constexpr T lo = std::numeric_limits<T>::min();
        const T x = static_cast<const T *>(o.p[0])[off[0]];
        if (x == lo) {
            out[i] = 0;
            return fail_key(seq, i, kOverflow);
        }
        out[i] = (op == CHELIS_INT_NEG || x < 0) ? (T)-x : x;
        return 0ull;
    }
};

// After a shift launch, in stream order: when the record names this
// launch's failure, the count at the failing element goes to the detail word
// (the C lane's message prints it). One thread; broadcast axes of the count
// have extent 1 and contribute nothing.
template <typename T>
__global__ void shift_detail_kernel(const unsigned long long *rec, uint64_t seq, Ops o, Shape sh, long long *detail) {
    if (threadIdx.x != 0) return;
    const unsigned long long w = __hip_atomic_load(rec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!w || ((~w) >> kSeqShift) != (seq >> kSeqShift)) return;
    const int64_t i = (int64_t)(((~w) >> 2) & ((1ull << (kSeqShift - 2)) - 1));
    int64_t off[2];
    offsets(o, sh, i, off);
    *detail = (long long)static_cast<const T *>(o.p[1])[off[1]];
}

// ---------------------------------------------------------------- gather
// A view's element at a row-major logical index (chelis_logical_offset).
struct View8 {
    int32_t rank;
    int32_t dense;
    int64_t shape[8], strides[8];
};
__device__ inline int64_t logical_offset(const View8 &v, int64_t i) {
    if (v.dense) return i;
    int64_t off = 0;
#pragma unroll
    for (int a = 7; a >= 0; --a) {
        if (a < v.rank) {
            off += (i % v.shape[a]) * v.strides[a];
            i /= v.shape[a];
        }
    }
    return off;
}
struct GatherGeom {
    int64_t axis_size, after, index_count, outer_per_batch, total;
};
// emit.rs:3807-3842 / kernels.rs:2557-2597: result element (b, j, d) of
// [before, index_count, after] reads values (b, g, d), g the index at
// (batch of b, j); an index outside [0, axis_size) fails (domain).
template <typename U, typename I>
__global__ __launch_bounds__(256) void gather_kernel(const U *__restrict__ values, View8 vv,
                                                     const I *__restrict__ idx, View8 iv, U *__restrict__ out,
                                                     GatherGeom g, uint64_t seq, unsigned long long *rec) {
    const int64_t stride = (int64_t)gridDim.x * kSelectThreads;
    for (int64_t base = (int64_t)blockIdx.x * kSelectThreads; base < g.total; base += stride) {
        const int64_t i = base + threadIdx.x;
        unsigned long long k = 0ull;
        if (i < g.total) {
            const int64_t d = i % g.after, t = i / g.after;
            const int64_t j = t % g.index_count, b = t / g.index_count;
            const int64_t pos = (b / g.outer_per_batch) * g.index_count + j;
            const int64_t x = (int64_t)idx[logical_offset(iv, pos)];
            if (x < 0 || x >= g.axis_size) {
                out[i] = U{};
                k = fail_key(seq, i, kDomain);
            } else {
                out[i] = values[logical_offset(vv, (b * g.axis_size + x) * g.after + d)];
            }
        }
        merge_failures(k, rec);
    }
}

// ---------------------------------------------------------------- ordered scan
// [05-OP-33] cumsum (kernels.rs:2793 ordered_scan, with the C lane's
// accumulation, crates/chelis-runtime/src/lib.rs:7020-7105): one thread per
// scan line of the [outer, n, inner] view - adjacent threads on adjacent
// inner positions, so the loads of a step are coalesced when inner is wide -
// walking its n leaves in order (from the end when reverse). The first leaf
// is the first prefix; each later prefix adds the leaf at the accumulator
// width (binary32 for bf16 / f16, i32 for i8 / i16); every prefix is stored
// at the result dtype, NaN canonical. An integer prefix outside the
// accumulator's range fails overflow, keyed by its place in the C lane's
// evaluation order (line by line, then step): ((o * inner + j) * n + step);
// the line then stores zeros.
template <int DT> struct ScanTypes { using A = float; using R = typename Dt<DT>::S; };
template <> struct ScanTypes<CHELIS_DTYPE_F64> { using A = double; using R = double; };
template <> struct ScanTypes<CHELIS_DTYPE_I8> { using A = int32_t; using R = int32_t; };
template <> struct ScanTypes<CHELIS_DTYPE_I16> { using A = int32_t; using R = int32_t; };
template <> struct ScanTypes<CHELIS_DTYPE_I32> { using A = int32_t; using R = int32_t; };
template <> struct ScanTypes<CHELIS_DTYPE_I64> { using A = int64_t; using R = int64_t; };

template <int DT>
__global__ __launch_bounds__(256) void cumsum_kernel(const typename Dt<DT>::S *__restrict__ x, View8 xv,
                                                     typename ScanTypes<DT>::R *__restrict__ y, int64_t outer,
                                                     int64_t n, int64_t inner, int reverse, uint64_t seq,
                                                     unsigned long long *rec) {
    using A = typename ScanTypes<DT>::A;
    using R = typename ScanTypes<DT>::R;
    const int64_t lines = outer * inner, stride = (int64_t)gridDim.x * kSelectThreads;
    for (int64_t base = (int64_t)blockIdx.x * kSelectThreads; base < lines; base += stride) {
        const int64_t t = base + threadIdx.x;
        unsigned long long k = 0ull;
        if (t < lines) {
            const int64_t o = t / inner, j = t % inner;
            A acc = A(0);
            bool failed = false;
            for (int64_t step = 0; step < n; ++step) {
                const int64_t pos = reverse ? n - 1 - step : step;
                const int64_t f = (o * n + pos) * inner + j;
                const typename Dt<DT>::S raw = x[logical_offset(xv, f)];
                if constexpr (Dt<DT>::kFloat) {
                    const A v = (A)semantic<DT>(raw);
                    acc = canon(step == 0 ? v : acc + v);
                    if constexpr (DT == CHELIS_DTYPE_BF16) y[f] = f32_to_bf16(acc);
                    else if constexpr (DT == CHELIS_DTYPE_F16) y[f] = f32_to_f16(acc);
                    else y[f] = acc;
                } else {
                    const A v = (A)raw;
                    A r = v;
                    if (!failed && step > 0 && __builtin_add_overflow(acc, v, &r)) {
                        failed = true;
                        k = fail_key(seq, t * n + step, kOverflow);
                    }
                    acc = failed ? A(0) : r;
                    y[f] = (R)acc;
                }
            }
        }
        if constexpr (!Dt<DT>::kFloat) merge_failures(k, rec);
    }
}

// ---------------------------------------------------------------- pad
// kernels.rs:1587-1637 / the C lane's emit_pad: output element o reads the
// source at o - lo on every axis when that lies inside the source, else it
// is the fill. Both sides strided (rank <= 8); elements moved as raw bits.
struct PadGeom {
    int32_t rank;
    int64_t out_shape[8], out_strides[8], lo[8], src_shape[8], src_strides[8];
};
template <typename U>
__global__ __launch_bounds__(256) void pad_kernel(const U *__restrict__ x, U *__restrict__ y, PadGeom g,
                                                  int64_t total, U fill) {
    const int64_t stride = (int64_t)gridDim.x * kSelectThreads;
    for (int64_t i = (int64_t)blockIdx.x * kSelectThreads + threadIdx.x; i < total; i += stride) {
        int64_t r = i, so = 0, yo = 0;
        bool inside = true;
#pragma unroll
        for (int a = 7; a >= 0; --a) {
            if (a < g.rank) {
                const int64_t c = r % g.out_shape[a];
                r /= g.out_shape[a];
                const int64_t sc = c - g.lo[a];
                inside = inside && sc >= 0 && sc < g.src_shape[a];
                so += sc * g.src_strides[a];
                yo += c * g.out_strides[a];
            }
        }
        U v = fill;
        if (inside) v = x[so];
        y[yo] = v;
    }
}

// ---------------------------------------------------------------- scatter
// ScatterAdd / Scatter / ScatterElements with the C lane's results
// (crates/chelis-backend-c/src/emit.rs:7382-7470, 7772-7990): every update
// gets its destination in the row-major target, then the (destination,
// position) pairs are radix-sorted - a stable sort, so each destination's
// updates lie together in ascending position. Scatter and ScatterElements
// keep the last of each run (the highest position: the last write); the
// add folds each run - the target's value, then the updates in order - by
// the canonical pair tree. The reference HIP lane adds with atomics (an
// order that varies run to run) and runs the replacing forms on one thread
// (crates/chelis-backend-hip/src/kernels.rs:2599-2765).
struct ScatterGeom {
    int64_t axis_size, after, index_count, outer_per_batch, total;  // hyperplane form
    int32_t elements, rank, axis;                                  // ScatterElements
    int64_t idx_shape[8], target_shape[8];
};

// An update's destination (the sentinel, past every destination, when its
// index is outside the axis: it fails domain at its position) and its
// position.
template <typename I, typename K>
__global__ __launch_bounds__(256) void scatter_keys_kernel(const I *__restrict__ indices, View8 iv, ScatterGeom g,
                                                           K sentinel, K *__restrict__ keys, K *__restrict__ pos,
                                                           uint64_t seq, unsigned long long *rec) {
    const int64_t stride = (int64_t)gridDim.x * kSelectThreads;
    for (int64_t base = (int64_t)blockIdx.x * kSelectThreads; base < g.total; base += stride) {
        const int64_t i = base + threadIdx.x;
        unsigned long long k = 0ull;
        if (i < g.total) {
            int64_t dst = 0;
            bool ok;
            if (g.elements) {
                const int64_t sel = (int64_t)indices[logical_offset(iv, i)];
                ok = sel >= 0 && sel < g.target_shape[g.axis];
                int64_t r = i, scale = 1;
                for (int a = g.rank - 1; a >= 0; --a) {
                    const int64_t c = r % g.idx_shape[a];
                    r /= g.idx_shape[a];
                    dst += (a == g.axis ? sel : c) * scale;
                    scale *= g.target_shape[a];
                }
            } else {
                const int64_t d = i % g.after, t = i / g.after, j = t % g.index_count, b = t / g.index_count;
                const int64_t sel = (int64_t)indices[logical_offset(iv, (b / g.outer_per_batch) * g.index_count + j)];
                ok = sel >= 0 && sel < g.axis_size;
                dst = (b * g.axis_size + sel) * g.after + d;
            }
            keys[i] = ok ? (K)dst : sentinel;
            pos[i] = (K)i;
            if (!ok) k = fail_key(seq, i, kDomain);
        }
        merge_failures(k, rec);
    }
}

// The last update of each destination's run.
template <typename U, typename K>
__global__ __launch_bounds__(256) void scatter_last_kernel(const K *__restrict__ skeys, const K *__restrict__ spos,
                                                           int64_t n, K sentinel, const U *__restrict__ upd, View8 uv,
                                                           U *__restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * kSelectThreads;
    for (int64_t p = (int64_t)blockIdx.x * kSelectThreads + threadIdx.x; p < n; p += stride) {
        const K d = skeys[p];
        if (d != sentinel && (p + 1 == n || skeys[p + 1] != d)) out[d] = upd[logical_offset(uv, (int64_t)spos[p])];
    }
}

// One node of the add's tree at the operand's arithmetic width: binary32 /
// binary64 adds; bf16 / f16 in binary32, rounded to the format at every
// node ([04-NUM-8]); integers checked against the width.
template <int DT>
struct AddNode {
    using S = typename Dt<DT>::S;
    using A = std::conditional_t<DT == CHELIS_DTYPE_F64, double,
                                 std::conditional_t<Dt<DT>::kFloat, float, int64_t>>;
    __device__ static A leaf(S v) {
        if constexpr (DT == CHELIS_DTYPE_BF16) return bf16_to_f32(v);
        else if constexpr (DT == CHELIS_DTYPE_F16) return f16_to_f32(v);
        else return (A)v;
    }
    __device__ static bool add(A l, A r, A *o) {
        if constexpr (DT == CHELIS_DTYPE_BF16) *o = bf16_to_f32(f32_to_bf16(l + r));
        else if constexpr (DT == CHELIS_DTYPE_F16) *o = f16_to_f32(f32_to_f16(l + r));
        else if constexpr (Dt<DT>::kFloat) *o = l + r;
        else {
            if (__builtin_add_overflow(l, r, o)) return false;
            return *o >= (A)std::numeric_limits<S>::min() && *o <= (A)std::numeric_limits<S>::max();
        }
        return true;
    }
    __device__ static S store(A v) {
        if constexpr (DT == CHELIS_DTYPE_BF16) return f32_to_bf16(v);
        else if constexpr (DT == CHELIS_DTYPE_F16) return f32_to_f16(v);
        else if constexpr (Dt<DT>::kFloat) return canon(v);
        else return (S)v;
    }
};

// A thread per run start folds [out[d], its updates...] leaf by leaf in a
// carry stack: a complete pair subtree of 2^l leaves waits at level l until
// its sibling arrives, and the partial subtrees left at the end join from
// the lowest level up - the canonical adjacent-pair tree. An integer node
// outside the width fails overflow, keyed past every update position (index
// errors come first, as in the C lane's order).
template <int DT, typename K>
__global__ __launch_bounds__(256) void scatter_add_kernel(const K *__restrict__ skeys, const K *__restrict__ spos,
                                                          int64_t n, K sentinel, const typename Dt<DT>::S *upd,
                                                          View8 uv, typename Dt<DT>::S *out, uint64_t seq,
                                                          unsigned long long *rec) {
    using N = AddNode<DT>;
    using A = typename N::A;
    const int64_t stride = (int64_t)gridDim.x * kSelectThreads;
    for (int64_t base = (int64_t)blockIdx.x * kSelectThreads; base < n; base += stride) {
        const int64_t p = base + threadIdx.x;
        unsigned long long k = 0ull;
        if (p < n) {
            const K d = skeys[p];
            if (d != sentinel && (p == 0 || skeys[p - 1] != d)) {
                A st[48];
                uint64_t cnt = 0;
                bool ok = true;
                auto push = [&](A v) {
                    int lv = 0;
                    for (uint64_t c = cnt; (c & 1) && ok; c >>= 1, ++lv) ok = N::add(st[lv], v, &v);
                    st[lv] = v;
                    ++cnt;
                };
                push(N::leaf(out[d]));
                for (int64_t q = p; q < n && skeys[q] == d && ok; ++q)
                    push(N::leaf(upd[logical_offset(uv, (int64_t)spos[q])]));
                A acc{};
                bool have = false;
                for (int lv = 0; ok && (cnt >> lv) != 0; ++lv)
                    if ((cnt >> lv) & 1) {
                        if (have) ok = N::add(st[lv], acc, &acc);
                        else acc = st[lv];
                        have = true;
                    }
                if (ok) out[d] = N::store(acc);
                else k = fail_key(seq, n + (int64_t)d, kOverflow);
            }
        }
        if constexpr (!Dt<DT>::kFloat) merge_failures(k, rec);
    }
}

// ---------------------------------------------------------------- host: the failure channel
// Per device: word [2..3] of the status words is the deferred record, [4..5]
// the record of a call that waits for its own result. A deferred launch's
// sequence number indexes the label ("add at i64") its message names.
constexpr int kMaxDevices = 64;
constexpr uint64_t kSeqMax = (1ull << (64 - kSeqShift)) - 1;
std::mutex g_fail_mutex;

struct Sink {
    unsigned long long *rec = nullptr;
    long long *detail = nullptr;  // a failing shift's count
    uint64_t seq = 0;
    bool wait = false;
};

// A deferred launch's message: "numeric trap: <kind> in <text>", or for a
// shift the C lane's count line.
struct Label {
    std::string text;
    bool shift = false;
    std::string overflow;  // when set, the text of an overflow (another prim)
};
std::vector<Label> g_labels[kMaxDevices];

const char *dtype_name(chelis_dtype d) {
    switch (d) {
        case CHELIS_DTYPE_F32: return "f32";
        case CHELIS_DTYPE_F64: return "f64";
        case CHELIS_DTYPE_I32: return "i32";
        case CHELIS_DTYPE_BOOL: return "bool";
        case CHELIS_DTYPE_I64: return "i64";
        case CHELIS_DTYPE_BF16: return "bf16";
        case CHELIS_DTYPE_F16: return "f16";
        case CHELIS_DTYPE_I8: return "i8";
        case CHELIS_DTYPE_I16: return "i16";
        default: return "key";
    }
}
const char *kind_text(int kind) {
    return kind == kOverflow ? "overflow" : kind == kDomain ? "domain" : "division by zero";
}

// The sink a trapping launch records into: its own word when the caller
// waits for the result (failure != NULL), else the deferred word under the
// next sequence number, labelled "<op> at <prim>".
int32_t open_sink(bool wait, const std::string &label, Sink *s, bool shift = false,
                  const std::string &overflow = std::string()) {
    int32_t *words = status_words(nullptr);
    if (!words) return set_error(CHELIS_HIP_EHIP, "no HIP device status words");
    s->wait = wait;
    if (wait) {
        s->rec = reinterpret_cast<unsigned long long *>(words + 4);
        s->detail = reinterpret_cast<long long *>(words + 8);
        s->seq = 0;
        return CHELIS_HIP_OK;
    }
    int device = 0;
    CHELIS_HIP_TRY(hipGetDevice(&device));
    std::lock_guard<std::mutex> lock(g_fail_mutex);
    std::vector<Label> &labels = g_labels[device];
    const uint64_t seq = std::min<uint64_t>(labels.size(), kSeqMax);
    if (labels.size() <= kSeqMax) labels.push_back(Label{label, shift, overflow});
    s->rec = reinterpret_cast<unsigned long long *>(words + 2);
    s->detail = reinterpret_cast<long long *>(words + 6);
    s->seq = seq << kSeqShift;
    return CHELIS_HIP_OK;
}

// The failure of a record word; a shift's message reads the count from the
// detail word (the stream is idle).
int32_t fill_failure(chelis_hip_numeric_failure *f, unsigned long long word, const Label &label,
                     const long long *detail) {
    f->index = -1;
    f->kind = 0;
    f->reserved = 0;
    f->message[0] = 0;
    if (!word) return CHELIS_HIP_OK;
    const uint64_t key = ~word;
    f->kind = (int32_t)(key & 3u);
    f->index = (int64_t)((key >> 2) & ((1ull << (kSeqShift - 2)) - 1));
    if (label.shift) {
        long long count = 0;
        CHELIS_HIP_TRY(hipMemcpy(&count, detail, sizeof count, hipMemcpyDeviceToHost));
        snprintf(f->message, sizeof f->message, "shift amount must be non-negative, got %lld", count);
    } else {
        const std::string &t = f->kind == kOverflow && !label.overflow.empty() ? label.overflow : label.text;
        snprintf(f->message, sizeof f->message, "numeric trap: %s in %s", kind_text(f->kind), t.c_str());
    }
    return CHELIS_HIP_OK;
}

// Reads and clears a record word (the stream is idle).
int32_t take_word(unsigned long long *rec, unsigned long long *word) {
    CHELIS_HIP_TRY(hipMemcpy(word, rec, sizeof *word, hipMemcpyDeviceToHost));
    if (*word) {
        const unsigned long long zero = 0ull;
        CHELIS_HIP_TRY(hipMemcpy(rec, &zero, sizeof zero, hipMemcpyHostToDevice));
    }
    return CHELIS_HIP_OK;
}

// After the launch of a waiting call: its record, read and cleared.
int32_t close_sink(const Sink &s, const std::string &label, chelis_hip_numeric_failure *f, bool shift = false,
                   const std::string &overflow = std::string()) {
    if (!s.wait) return CHELIS_HIP_OK;
    CHELIS_HIP_TRY(hipStreamSynchronize(stream()));
    unsigned long long word = 0ull;
    if (int32_t st = take_word(s.rec, &word)) return st;
    return fill_failure(f, word, Label{label, shift, overflow}, s.detail);
}

// ---------------------------------------------------------------- host: checks and launches
int32_t check_broadcast(const chelis_gpu_tensor *in, const chelis_gpu_tensor *out, const char *what,
                        const char *name) {
    if (int32_t s = check_tensor(in, name)) return s;
    if (in->rank != out->rank) return set_error(CHELIS_HIP_EDOMAIN, "%s: %s rank differs from the output", what, name);
    for (int32_t a = 0; a < in->rank; ++a)
        if (in->shape[a] != out->shape[a] && in->shape[a] != 1)
            return set_error(CHELIS_HIP_EDOMAIN, "%s: %s axis %d neither matches nor broadcasts", what, name, a);
    return CHELIS_HIP_OK;
}

int32_t check_out(const chelis_gpu_tensor *out, const char *what) {
    if (int32_t s = check_tensor(out, "out")) return s;
    if (!is_contiguous(out)) return set_error(CHELIS_HIP_EUNSUPPORTED, "%s: the output must be contiguous", what);
    return CHELIS_HIP_OK;
}

// A strided output no two of whose elements share an address: sorted by
// stride, each axis steps past everything the smaller axes span.
bool non_overlapping(const chelis_gpu_tensor *t) {
    std::vector<std::pair<int64_t, int64_t>> ax;
    for (int32_t a = 0; a < t->rank; ++a)
        if (t->shape[a] > 1) ax.push_back({t->strides[a], t->shape[a]});
    std::sort(ax.begin(), ax.end());
    int64_t span = 1;
    for (const auto &p : ax) {
        if (p.first < span) return false;
        span = p.first * p.second;
    }
    return true;
}

int64_t map_blocks(int64_t count) { return std::max<int64_t>(1, std::min<int64_t>((count + 255) / 256, 65536)); }

template <class F>
int32_t launch_map(const F &f, const chelis_gpu_tensor *const *ins, int n, const chelis_gpu_tensor *out,
                   unsigned long long *rec, const char *what) {
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    if (!out->count) return CHELIS_HIP_OK;
    Shape sh;
    int64_t s[CHELIS_FUSED_MAX_INPUTS][kMaxRank] = {};
    if (!collapse(out, ins, n, &sh, s))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "%s: more than %d independent axes", what, kMaxRank);
    Ops o{};
    for (int k = 0; k < n; ++k) {
        o.p[k] = ins[k]->data;
        for (int a = 0; a < kMaxRank; ++a) o.st[k][a] = s[k][a];
    }
    map_kernel<F><<<dim3((unsigned)map_blocks(out->count)), dim3(256), 0, st>>>(f, o, sh, out->count, rec);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

template <int DT>
int32_t launch_compare(int32_t kind, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                       const chelis_gpu_tensor *out) {
    const chelis_gpu_tensor *ins[2] = {a, b};
    return launch_map(CompareOp<DT>{kind, static_cast<uint8_t *>(out->data)}, ins, 2, out, nullptr, "compare");
}

template <int SRC, int DST>
int32_t launch_cast(const chelis_gpu_tensor *x, const chelis_gpu_tensor *out, const Sink &s) {
    const chelis_gpu_tensor *ins[1] = {x};
    return launch_map(CastOp<SRC, DST>{static_cast<typename Dt<DST>::S *>(out->data), s.seq}, ins, 1, out, s.rec,
                      "cast");
}

template <int SRC>
int32_t cast_to(chelis_dtype dst, const chelis_gpu_tensor *x, const chelis_gpu_tensor *out, const Sink &s) {
    switch (dst) {
        case CHELIS_DTYPE_F32: return launch_cast<SRC, CHELIS_DTYPE_F32>(x, out, s);
        case CHELIS_DTYPE_F64: return launch_cast<SRC, CHELIS_DTYPE_F64>(x, out, s);
        case CHELIS_DTYPE_BF16: return launch_cast<SRC, CHELIS_DTYPE_BF16>(x, out, s);
        case CHELIS_DTYPE_F16: return launch_cast<SRC, CHELIS_DTYPE_F16>(x, out, s);
        case CHELIS_DTYPE_I8: return launch_cast<SRC, CHELIS_DTYPE_I8>(x, out, s);
        case CHELIS_DTYPE_I16: return launch_cast<SRC, CHELIS_DTYPE_I16>(x, out, s);
        case CHELIS_DTYPE_I32: return launch_cast<SRC, CHELIS_DTYPE_I32>(x, out, s);
        case CHELIS_DTYPE_I64: return launch_cast<SRC, CHELIS_DTYPE_I64>(x, out, s);
        case CHELIS_DTYPE_BOOL: return launch_cast<SRC, CHELIS_DTYPE_BOOL>(x, out, s);
        default: return set_error(CHELIS_HIP_EUNSUPPORTED, "cast: no target dtype %d", (int)dst);
    }
}

bool is_int(chelis_dtype d) {
    return d == CHELIS_DTYPE_I8 || d == CHELIS_DTYPE_I16 || d == CHELIS_DTYPE_I32 || d == CHELIS_DTYPE_I64;
}
bool is_castable(chelis_dtype d) { return is_int(d) || is_float(d) || is_narrow16(d) || d == CHELIS_DTYPE_BOOL; }

template <typename T>
int32_t launch_int(int32_t op, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, const chelis_gpu_tensor *out,
                   const Sink &s) {
    T *o = static_cast<T *>(out->data);
    if (op == CHELIS_INT_NEG || op == CHELIS_INT_ABS) {
        const chelis_gpu_tensor *ins[1] = {a};
        return launch_map(IntUnaryOp<T>{op, o, s.seq}, ins, 1, out, s.rec, "integer_elementwise");
    }
    const chelis_gpu_tensor *ins[2] = {a, b};
    if (int32_t st = launch_map(IntBinaryOp<T>{op, o, s.seq}, ins, 2, out, s.rec, "integer_elementwise")) return st;
    if ((op == CHELIS_INT_SHL || op == CHELIS_INT_SHR) && out->count) {
        Shape sh;
        int64_t st2[CHELIS_FUSED_MAX_INPUTS][kMaxRank] = {};
        collapse(out, ins, 2, &sh, st2);  // succeeded in launch_map
        Ops ops{};
        for (int k = 0; k < 2; ++k) {
            ops.p[k] = ins[k]->data;
            for (int ax = 0; ax < kMaxRank; ++ax) ops.st[k][ax] = st2[k][ax];
        }
        shift_detail_kernel<T><<<1, 64, 0, stream()>>>(s.rec, s.seq, ops, sh, s.detail);
        CHELIS_LAUNCH_CHECK();
    }
    return CHELIS_HIP_OK;
}

const char *int_op_name(int32_t op) {
    static const char *names[] = {"add",      "sub",      "mul", "floor_div", "trunc_div", "mod",    "max_elem",
                                  "min_elem", "neg",      "abs", "bitand",    "bitor",     "bitxor", "shl",
                                  "shr"};
    return op >= 0 && op <= CHELIS_INT_SHR ? names[op] : "?";
}

View8 view_of(const chelis_gpu_tensor *t) {
    View8 v{};
    v.rank = t->rank;
    v.dense = is_contiguous(t) ? 1 : 0;
    for (int32_t a = 0; a < t->rank; ++a) {
        v.shape[a] = t->shape[a];
        v.strides[a] = t->strides[a];
    }
    return v;
}

template <typename U>
int32_t launch_gather(const chelis_gpu_tensor *values, const chelis_gpu_tensor *indices, const chelis_gpu_tensor *out,
                      const GatherGeom &g, const Sink &s) {
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    if (!g.total) return CHELIS_HIP_OK;
    const unsigned blocks = (unsigned)map_blocks(g.total);
    if (indices->dtype == CHELIS_DTYPE_I32)
        gather_kernel<U, int32_t><<<dim3(blocks), dim3(256), 0, st>>>(
            static_cast<const U *>(values->data), view_of(values), static_cast<const int32_t *>(indices->data),
            view_of(indices), static_cast<U *>(out->data), g, s.seq, s.rec);
    else
        gather_kernel<U, int64_t><<<dim3(blocks), dim3(256), 0, st>>>(
            static_cast<const U *>(values->data), view_of(values), static_cast<const int64_t *>(indices->data),
            view_of(indices), static_cast<U *>(out->data), g, s.seq, s.rec);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

}  // namespace

// ---------------------------------------------------------------- C ABI
extern "C" int32_t chelis_hip_compare(int32_t kind, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                                      const chelis_gpu_tensor *out) {
    if (int32_t s = check_out(out, "compare")) return s;
    if (out->dtype != CHELIS_DTYPE_BOOL) return set_error(CHELIS_HIP_EDOMAIN, "compare: the output must be bool");
    if (kind < CHELIS_CMP_CMPLT || kind > CHELIS_CMP_LTE)
        return set_error(CHELIS_HIP_EDOMAIN, "compare: unknown kind %d", kind);
    if (int32_t s = check_broadcast(a, out, "compare", "a")) return s;
    if (int32_t s = check_broadcast(b, out, "compare", "b")) return s;
    if (a->dtype != b->dtype) return set_error(CHELIS_HIP_EDOMAIN, "compare: operand dtypes differ");
    switch (a->dtype) {
        case CHELIS_DTYPE_F32: return launch_compare<CHELIS_DTYPE_F32>(kind, a, b, out);
        case CHELIS_DTYPE_F64: return launch_compare<CHELIS_DTYPE_F64>(kind, a, b, out);
        case CHELIS_DTYPE_BF16: return launch_compare<CHELIS_DTYPE_BF16>(kind, a, b, out);
        case CHELIS_DTYPE_F16: return launch_compare<CHELIS_DTYPE_F16>(kind, a, b, out);
        case CHELIS_DTYPE_I8: return launch_compare<CHELIS_DTYPE_I8>(kind, a, b, out);
        case CHELIS_DTYPE_I16: return launch_compare<CHELIS_DTYPE_I16>(kind, a, b, out);
        case CHELIS_DTYPE_I32: return launch_compare<CHELIS_DTYPE_I32>(kind, a, b, out);
        case CHELIS_DTYPE_I64: return launch_compare<CHELIS_DTYPE_I64>(kind, a, b, out);
        case CHELIS_DTYPE_BOOL:
            if (kind != CHELIS_CMP_EQ && kind != CHELIS_CMP_NEQ)
                return set_error(CHELIS_HIP_EDOMAIN, "compare: bool admits eq and neq only");
            return launch_compare<CHELIS_DTYPE_BOOL>(kind, a, b, out);
        default: return set_error(CHELIS_HIP_EUNSUPPORTED, "compare: no dtype %d", (int)a->dtype);
    }
}

extern "C" int32_t chelis_hip_logical(int32_t kind, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                                      const chelis_gpu_tensor *out) {
    if (int32_t s = check_out(out, "logical")) return s;
    if (kind < CHELIS_LOGICAL_AND || kind > CHELIS_LOGICAL_NOT)
        return set_error(CHELIS_HIP_EDOMAIN, "logical: unknown kind %d", kind);
    if (kind == CHELIS_LOGICAL_NOT) b = a;
    if (int32_t s = check_broadcast(a, out, "logical", "a")) return s;
    if (int32_t s = check_broadcast(b, out, "logical", "b")) return s;
    if (a->dtype != CHELIS_DTYPE_BOOL || b->dtype != CHELIS_DTYPE_BOOL || out->dtype != CHELIS_DTYPE_BOOL)
        return set_error(CHELIS_HIP_EDOMAIN, "logical: operands and output must be bool");
    const chelis_gpu_tensor *ins[2] = {a, b};
    return launch_map(LogicalOp{kind, static_cast<uint8_t *>(out->data)}, ins, 2, out, nullptr, "logical");
}

extern "C" int32_t chelis_hip_where(const chelis_gpu_tensor *cond, const chelis_gpu_tensor *a,
                                    const chelis_gpu_tensor *b, const chelis_gpu_tensor *out) {
    if (int32_t s = check_out(out, "where")) return s;
    if (int32_t s = check_broadcast(cond, out, "where", "cond")) return s;
    if (int32_t s = check_broadcast(a, out, "where", "a")) return s;
    if (int32_t s = check_broadcast(b, out, "where", "b")) return s;
    if (cond->dtype != CHELIS_DTYPE_BOOL) return set_error(CHELIS_HIP_EDOMAIN, "where: the condition must be bool");
    if (a->dtype != out->dtype || b->dtype != out->dtype)
        return set_error(CHELIS_HIP_EDOMAIN, "where: branch dtypes differ from the output");
    const chelis_gpu_tensor *ins[3] = {cond, a, b};
    switch (dtype_width(out->dtype)) {
        case 1: return launch_map(WhereOp<uint8_t>{static_cast<uint8_t *>(out->data)}, ins, 3, out, nullptr, "where");
        case 2: return launch_map(WhereOp<uint16_t>{static_cast<uint16_t *>(out->data)}, ins, 3, out, nullptr, "where");
        case 4: return launch_map(WhereOp<uint32_t>{static_cast<uint32_t *>(out->data)}, ins, 3, out, nullptr, "where");
        default:
            return launch_map(WhereOp<uint64_t>{static_cast<uint64_t *>(out->data)}, ins, 3, out, nullptr, "where");
    }
}

extern "C" int32_t chelis_hip_extrema_adjoint(int32_t kind, int32_t operand, const chelis_gpu_tensor *a,
                                              const chelis_gpu_tensor *b, const chelis_gpu_tensor *g,
                                              const chelis_gpu_tensor *out) {
    if (int32_t s = check_out(out, "extrema_adjoint")) return s;
    if ((kind != CHELIS_EXTREMA_MAX && kind != CHELIS_EXTREMA_MIN) ||
        (operand != CHELIS_EXTREMA_LEFT && operand != CHELIS_EXTREMA_RIGHT))
        return set_error(CHELIS_HIP_EDOMAIN, "extrema_adjoint: unknown kind %d or operand %d", kind, operand);
    if (int32_t s = check_broadcast(a, out, "extrema_adjoint", "a")) return s;
    if (int32_t s = check_broadcast(b, out, "extrema_adjoint", "b")) return s;
    if (int32_t s = check_broadcast(g, out, "extrema_adjoint", "g")) return s;
    if (a->dtype != out->dtype || b->dtype != out->dtype || g->dtype != out->dtype)
        return set_error(CHELIS_HIP_EDOMAIN, "extrema_adjoint: operand dtypes differ from the output");
    const chelis_gpu_tensor *ins[3] = {a, b, g};
    const int32_t mn = kind == CHELIS_EXTREMA_MIN, rt = operand == CHELIS_EXTREMA_RIGHT;
    switch (out->dtype) {
        case CHELIS_DTYPE_F32:
            return launch_map(ExtremaAdjointOp<CHELIS_DTYPE_F32>{mn, rt, static_cast<float *>(out->data)}, ins, 3,
                              out, nullptr, "extrema_adjoint");
        case CHELIS_DTYPE_F64:
            return launch_map(ExtremaAdjointOp<CHELIS_DTYPE_F64>{mn, rt, static_cast<double *>(out->data)}, ins, 3,
                              out, nullptr, "extrema_adjoint");
        case CHELIS_DTYPE_BF16:
            return launch_map(ExtremaAdjointOp<CHELIS_DTYPE_BF16>{mn, rt, static_cast<uint16_t *>(out->data)}, ins,
                              3, out, nullptr, "extrema_adjoint");
        case CHELIS_DTYPE_F16:
            return launch_map(ExtremaAdjointOp<CHELIS_DTYPE_F16>{mn, rt, static_cast<uint16_t *>(out->data)}, ins,
                              3, out, nullptr, "extrema_adjoint");
        default: return set_error(CHELIS_HIP_EUNSUPPORTED, "extrema_adjoint: f32, f64, bf16 or f16 only");
    }
}

extern "C" int32_t chelis_hip_cast(const chelis_gpu_tensor *x, const chelis_gpu_tensor *out,
                                   chelis_hip_numeric_failure *failure) {
    if (int32_t s = check_out(out, "cast")) return s;
    if (int32_t s = check_broadcast(x, out, "cast", "x")) return s;
    if (!is_castable(x->dtype) || !is_castable(out->dtype))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "cast: no cast from dtype %d to %d", (int)x->dtype,
                         (int)out->dtype);
    const std::string label = std::string("cast at ") + dtype_name(out->dtype);
    Sink sink;
    if (int32_t s = open_sink(failure != nullptr, label, &sink)) return s;
    int32_t st;
    switch (x->dtype) {
        case CHELIS_DTYPE_F32: st = cast_to<CHELIS_DTYPE_F32>(out->dtype, x, out, sink); break;
        case CHELIS_DTYPE_F64: st = cast_to<CHELIS_DTYPE_F64>(out->dtype, x, out, sink); break;
        case CHELIS_DTYPE_BF16: st = cast_to<CHELIS_DTYPE_BF16>(out->dtype, x, out, sink); break;
        case CHELIS_DTYPE_F16: st = cast_to<CHELIS_DTYPE_F16>(out->dtype, x, out, sink); break;
        case CHELIS_DTYPE_I8: st = cast_to<CHELIS_DTYPE_I8>(out->dtype, x, out, sink); break;
        case CHELIS_DTYPE_I16: st = cast_to<CHELIS_DTYPE_I16>(out->dtype, x, out, sink); break;
        case CHELIS_DTYPE_I32: st = cast_to<CHELIS_DTYPE_I32>(out->dtype, x, out, sink); break;
        case CHELIS_DTYPE_I64: st = cast_to<CHELIS_DTYPE_I64>(out->dtype, x, out, sink); break;
        default: st = cast_to<CHELIS_DTYPE_BOOL>(out->dtype, x, out, sink); break;
    }
    if (st) return st;
    return close_sink(sink, label, failure);
}

extern "C" int32_t chelis_hip_integer_elementwise(int32_t op, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                                                  const chelis_gpu_tensor *out, chelis_hip_numeric_failure *failure) {
    if (op < CHELIS_INT_ADD || op > CHELIS_INT_SHR)
        return set_error(CHELIS_HIP_EDOMAIN, "integer_elementwise: unknown op %d", op);
    const bool shift = op == CHELIS_INT_SHL || op == CHELIS_INT_SHR;
    const bool unary = op == CHELIS_INT_NEG || op == CHELIS_INT_ABS;
    if (int32_t s = check_out(out, "integer_elementwise")) return s;
    if (int32_t s = check_broadcast(a, out, "integer_elementwise", "a")) return s;
    if (!unary) {
        if (int32_t s = check_broadcast(b, out, "integer_elementwise", "b")) return s;
        if (b->dtype != out->dtype) return set_error(CHELIS_HIP_EDOMAIN, "integer_elementwise: b's dtype differs");
    }
    if (a->dtype != out->dtype) return set_error(CHELIS_HIP_EDOMAIN, "integer_elementwise: a's dtype differs");
    if (!is_int(out->dtype))
        return set_error(CHELIS_HIP_EDOMAIN, "integer_elementwise: i8, i16, i32 or i64 operands only");
    const std::string label = std::string(int_op_name(op)) + " at " + dtype_name(out->dtype);
    Sink sink;
    if (int32_t s = open_sink(failure != nullptr, label, &sink, shift)) return s;
    int32_t st;
    switch (out->dtype) {
        case CHELIS_DTYPE_I8: st = launch_int<int8_t>(op, a, b, out, sink); break;
        case CHELIS_DTYPE_I16: st = launch_int<int16_t>(op, a, b, out, sink); break;
        case CHELIS_DTYPE_I32: st = launch_int<int32_t>(op, a, b, out, sink); break;
        default: st = launch_int<int64_t>(op, a, b, out, sink); break;
    }
    if (st) return st;
    return close_sink(sink, label, failure, shift);
}

extern "C" int32_t chelis_hip_gather(const chelis_gpu_tensor *values, const chelis_gpu_tensor *indices, int32_t axis,
                                     int32_t batch_rank, const chelis_gpu_tensor *out,
                                     chelis_hip_numeric_failure *failure) {
    if (int32_t s = check_tensor(values, "values")) return s;
    if (int32_t s = check_tensor(indices, "indices")) return s;
    if (int32_t s = check_out(out, "gather")) return s;
    if (indices->dtype != CHELIS_DTYPE_I32 && indices->dtype != CHELIS_DTYPE_I64)
        return set_error(CHELIS_HIP_EDOMAIN, "gather: indices must be i32 or i64");
    if (out->dtype != values->dtype) return set_error(CHELIS_HIP_EDOMAIN, "gather: output dtype differs from values");
    if (axis < 0 || axis >= values->rank || batch_rank < 0 || batch_rank > axis || batch_rank > indices->rank)
        return set_error(CHELIS_HIP_EDOMAIN, "gather: axis %d / batch_rank %d outside the operands", axis, batch_rank);
    // the result is values[..axis] ++ indices[batch_rank..] ++ values[axis+1..]
    const int32_t want_rank = values->rank - 1 + indices->rank - batch_rank;
    bool shape_ok = out->rank == want_rank;
    for (int32_t a = 0, k = 0; shape_ok && a < values->rank; ++a) {
        if (a == axis) {
            for (int32_t q = batch_rank; q < indices->rank && shape_ok; ++q) shape_ok = out->shape[k++] == indices->shape[q];
        } else {
            shape_ok = out->shape[k++] == values->shape[a];
        }
    }
    if (!shape_ok) return set_error(CHELIS_HIP_EDOMAIN, "gather: output shape is not the gathered shape");
    // emit.rs:3829-3841: paired batch axes must agree (a domain trap)
    int64_t batch = 1, before = 1, after = 1;
    for (int32_t a = 0; a < batch_rank; ++a) {
        if (values->shape[a] != indices->shape[a])
            return set_error(CHELIS_HIP_EDOMAIN, "numeric trap: domain in gather at i64");
        batch *= values->shape[a];
    }
    for (int32_t a = 0; a < axis; ++a) before *= values->shape[a];
    for (int32_t a = axis + 1; a < values->rank; ++a) after *= values->shape[a];
    GatherGeom g{};
    g.axis_size = values->shape[axis];
    g.after = after;
    g.index_count = batch == 0 ? 0 : indices->count / batch;
    g.outer_per_batch = (batch == 0 || before == 0) ? 1 : before / batch;
    g.total = out->count;
    if (g.total && (g.after == 0 || g.index_count == 0)) g.total = 0;  // no element to read
    const std::string label = "gather at i64";
    Sink sink;
    if (int32_t s = open_sink(failure != nullptr, label, &sink)) return s;
    int32_t st;
    switch (dtype_width(values->dtype)) {
        case 1: st = launch_gather<uint8_t>(values, indices, out, g, sink); break;
        case 2: st = launch_gather<uint16_t>(values, indices, out, g, sink); break;
        case 4: st = launch_gather<uint32_t>(values, indices, out, g, sink); break;
        default: st = launch_gather<uint64_t>(values, indices, out, g, sink); break;
    }
    if (st) return st;
    return close_sink(sink, label, failure);
}

namespace {
template <int DT>
int32_t launch_cumsum(const chelis_gpu_tensor *x, const chelis_gpu_tensor *out, int64_t outer, int64_t n,
                      int64_t inner, int32_t reverse, const Sink &s) {
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    const int64_t lines = outer * inner;
    if (!lines || !n) return CHELIS_HIP_OK;
    cumsum_kernel<DT><<<dim3((unsigned)map_blocks(lines)), dim3(256), 0, st>>>(
        static_cast<const typename Dt<DT>::S *>(x->data), view_of(x),
        static_cast<typename ScanTypes<DT>::R *>(out->data), outer, n, inner, reverse, s.seq, s.rec);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}
}  // namespace

extern "C" int32_t chelis_hip_cumsum(const chelis_gpu_tensor *x, int32_t axis, int32_t reverse,
                                     const chelis_gpu_tensor *out, chelis_hip_numeric_failure *failure) {
    if (int32_t s = check_tensor(x, "x")) return s;
    if (int32_t s = check_out(out, "cumsum")) return s;
    if (x->dtype == CHELIS_DTYPE_BOOL || !is_castable(x->dtype))
        return set_error(CHELIS_HIP_EDOMAIN, "cumsum: a signed integer or float operand");
    if (axis < 0 || axis >= x->rank) return set_error(CHELIS_HIP_EDOMAIN, "cumsum: axis %d outside the rank", axis);
    const chelis_dtype rdt = (x->dtype == CHELIS_DTYPE_I8 || x->dtype == CHELIS_DTYPE_I16) ? CHELIS_DTYPE_I32 : x->dtype;
    if (out->dtype != rdt) return set_error(CHELIS_HIP_EDOMAIN, "cumsum: the result dtype is %s", dtype_name(rdt));
    if (!same_shape(x, out)) return set_error(CHELIS_HIP_EDOMAIN, "cumsum: the result has the operand's shape");
    int64_t outer = 1, inner = 1;
    for (int32_t a = 0; a < axis; ++a) outer *= x->shape[a];
    for (int32_t a = axis + 1; a < x->rank; ++a) inner *= x->shape[a];
    const int64_t n = x->shape[axis];
    const std::string label = std::string("cumsum at ") + dtype_name(rdt);
    Sink sink;
    if (int32_t s = open_sink(failure != nullptr, label, &sink)) return s;
    int32_t st;
    switch (x->dtype) {
        case CHELIS_DTYPE_F32: st = launch_cumsum<CHELIS_DTYPE_F32>(x, out, outer, n, inner, reverse, sink); break;
        case CHELIS_DTYPE_F64: st = launch_cumsum<CHELIS_DTYPE_F64>(x, out, outer, n, inner, reverse, sink); break;
        case CHELIS_DTYPE_BF16: st = launch_cumsum<CHELIS_DTYPE_BF16>(x, out, outer, n, inner, reverse, sink); break;
        case CHELIS_DTYPE_F16: st = launch_cumsum<CHELIS_DTYPE_F16>(x, out, outer, n, inner, reverse, sink); break;
        case CHELIS_DTYPE_I8: st = launch_cumsum<CHELIS_DTYPE_I8>(x, out, outer, n, inner, reverse, sink); break;
        case CHELIS_DTYPE_I16: st = launch_cumsum<CHELIS_DTYPE_I16>(x, out, outer, n, inner, reverse, sink); break;
        case CHELIS_DTYPE_I32: st = launch_cumsum<CHELIS_DTYPE_I32>(x, out, outer, n, inner, reverse, sink); break;
        default: st = launch_cumsum<CHELIS_DTYPE_I64>(x, out, outer, n, inner, reverse, sink); break;
    }
    if (st) return st;
    return close_sink(sink, label, failure);
}

template <typename U>
int32_t launch_pad(const chelis_gpu_tensor *x, const PadGeom &g, uint64_t fill, const chelis_gpu_tensor *out) {
    pad_kernel<U><<<dim3((unsigned)map_blocks(out->count)), dim3(256), 0, stream()>>>(
        static_cast<const U *>(x->data), static_cast<U *>(out->data), g, out->count, (U)fill);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

extern "C" int32_t chelis_hip_pad(const chelis_gpu_tensor *x, const int64_t *lo, uint64_t fill_bits,
                                  const chelis_gpu_tensor *out) {
    if (int32_t s = check_tensor(x, "x")) return s;
    if (int32_t s = check_tensor(out, "out")) return s;
    if (!non_overlapping(out)) return set_error(CHELIS_HIP_EUNSUPPORTED, "pad: the output's elements overlap");
    if (out->dtype != x->dtype) return set_error(CHELIS_HIP_EDOMAIN, "pad: output dtype differs from x");
    if (x->rank != out->rank || x->rank > 8)
        return set_error(CHELIS_HIP_EDOMAIN, "pad: x and the output need one rank, at most 8");
    if (x->rank > 0 && !lo) return set_error(CHELIS_HIP_EDOMAIN, "pad: null lo");
    PadGeom g{};
    g.rank = x->rank;
    for (int32_t a = 0; a < x->rank; ++a) {
        if (lo[a] < 0 || x->shape[a] < 0 || lo[a] + x->shape[a] > out->shape[a])
            return set_error(CHELIS_HIP_EDOMAIN, "pad: axis %d: %lld before %lld source elements exceed %lld", a,
                             (long long)lo[a], (long long)x->shape[a], (long long)out->shape[a]);
        g.out_shape[a] = out->shape[a];
        g.out_strides[a] = out->strides[a];
        g.lo[a] = lo[a];
        g.src_shape[a] = x->shape[a];
        g.src_strides[a] = x->strides[a];
    }
    if (!stream()) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    if (!out->count) return CHELIS_HIP_OK;
    switch (dtype_width(out->dtype)) {
        case 1: return launch_pad<uint8_t>(x, g, fill_bits, out);
        case 2: return launch_pad<uint16_t>(x, g, fill_bits, out);
        case 4: return launch_pad<uint32_t>(x, g, fill_bits, out);
        default: return launch_pad<uint64_t>(x, g, fill_bits, out);
    }
}

namespace {
// The scatter's passes over keys of width K (destinations and positions):
// the target copied into out, the keys, the stable sort, the runs applied.
template <typename K>
int32_t run_scatter(int32_t mode, const chelis_gpu_tensor *target, const chelis_gpu_tensor *indices,
                    const chelis_gpu_tensor *updates, const chelis_gpu_tensor *out, const ScatterGeom &g,
                    const Sink &s) {
    hipStream_t st = stream();
    const int64_t zeros[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (int32_t r = chelis_hip_pad(target, zeros, 0, out)) return r;
    const int64_t n = g.total;
    if (!n) return CHELIS_HIP_OK;
    const K sentinel = (K)out->count;
    int end_bit = 1;
    while (end_bit < (int)(8 * sizeof(K)) && ((uint64_t)sentinel >> end_bit) != 0) ++end_bit;
    size_t temp = 0;
    K *none = nullptr;
    // the item count hipcub takes is an int: a larger scatter is refused by the caller
    CHELIS_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, temp, none, none, none, none, (int)n, 0, end_bit, st));
    const size_t pairs = (size_t)n * sizeof(K);
    char *buf = static_cast<char *>(scratch_alloc(4 * pairs + temp));
    if (!buf) return set_error(CHELIS_HIP_EHIP, "scatter: no device memory for %lld updates", (long long)n);
    K *keys = reinterpret_cast<K *>(buf), *pos = keys + n, *skeys = pos + n, *spos = skeys + n;
    void *tmp = buf + 4 * pairs;
    int32_t rc = CHELIS_HIP_OK;
    const View8 iv = view_of(indices), uv = view_of(updates);
    const unsigned blocks = (unsigned)map_blocks(n);
    if (indices->dtype == CHELIS_DTYPE_I32)
        scatter_keys_kernel<int32_t, K><<<blocks, 256, 0, st>>>(static_cast<const int32_t *>(indices->data), iv, g,
                                                               sentinel, keys, pos, s.seq, s.rec);
    else
        scatter_keys_kernel<int64_t, K><<<blocks, 256, 0, st>>>(static_cast<const int64_t *>(indices->data), iv, g,
                                                               sentinel, keys, pos, s.seq, s.rec);
    if (hipGetLastError() != hipSuccess) rc = set_error(CHELIS_HIP_EHIP, "scatter: key launch failed");
    if (!rc && hipcub::DeviceRadixSort::SortPairs(tmp, temp, keys, skeys, pos, spos, (int)n, 0, end_bit, st) !=
                   hipSuccess)
        rc = set_error(CHELIS_HIP_EHIP, "scatter: the sort failed");
    if (!rc) {
        if (mode != 1) {
            switch (dtype_width(out->dtype)) {
                case 1:
                    scatter_last_kernel<uint8_t, K><<<blocks, 256, 0, st>>>(
                        skeys, spos, n, sentinel, static_cast<const uint8_t *>(updates->data), uv,
                        static_cast<uint8_t *>(out->data));
                    break;
                case 2:
                    scatter_last_kernel<uint16_t, K><<<blocks, 256, 0, st>>>(
                        skeys, spos, n, sentinel, static_cast<const uint16_t *>(updates->data), uv,
                        static_cast<uint16_t *>(out->data));
                    break;
                case 4:
                    scatter_last_kernel<uint32_t, K><<<blocks, 256, 0, st>>>(
                        skeys, spos, n, sentinel, static_cast<const uint32_t *>(updates->data), uv,
                        static_cast<uint32_t *>(out->data));
                    break;
                default:
                    scatter_last_kernel<uint64_t, K><<<blocks, 256, 0, st>>>(
                        skeys, spos, n, sentinel, static_cast<const uint64_t *>(updates->data), uv,
                        static_cast<uint64_t *>(out->data));
            }
        } else {
#define CHELIS_SCATTER_ADD(DT)                                                                                    \
    case DT:                                                                                                      \
        scatter_add_kernel<DT, K><<<blocks, 256, 0, st>>>(                                                        \
            skeys, spos, n, sentinel, static_cast<const typename Dt<DT>::S *>(updates->data), uv,                 \
            static_cast<typename Dt<DT>::S *>(out->data), s.seq, s.rec);                                          \
        break;
            switch (out->dtype) {
                CHELIS_SCATTER_ADD(CHELIS_DTYPE_F32)
                CHELIS_SCATTER_ADD(CHELIS_DTYPE_F64)
                CHELIS_SCATTER_ADD(CHELIS_DTYPE_BF16)
                CHELIS_SCATTER_ADD(CHELIS_DTYPE_F16)
                CHELIS_SCATTER_ADD(CHELIS_DTYPE_I8)
                CHELIS_SCATTER_ADD(CHELIS_DTYPE_I16)
                CHELIS_SCATTER_ADD(CHELIS_DTYPE_I32)
                CHELIS_SCATTER_ADD(CHELIS_DTYPE_I64)
                default: rc = set_error(CHELIS_HIP_EDOMAIN, "scatter: no add for this dtype");
            }
#undef CHELIS_SCATTER_ADD
        }
        if (!rc && hipGetLastError() != hipSuccess) rc = set_error(CHELIS_HIP_EHIP, "scatter: launch failed");
    }
    scratch_free(buf, 4 * pairs + temp);
    return rc;
}

int32_t scatter_common(int32_t mode, const chelis_gpu_tensor *target, const chelis_gpu_tensor *indices,
                       const chelis_gpu_tensor *updates, const chelis_gpu_tensor *out, ScatterGeom &g,
                       chelis_hip_numeric_failure *failure) {
    static const char *names[] = {"scatter_replace", "scatter", "scatter_elements"};
    const std::string label = std::string(names[mode]) + " at i64";
    const std::string overflow = mode == 1 ? std::string("scatter at ") + dtype_name(out->dtype) : std::string();
    if (g.total > (int64_t)std::numeric_limits<int>::max())
        return set_error(CHELIS_HIP_EUNSUPPORTED, "%s: more than 2^31 - 1 updates", names[mode]);
    Sink sink;
    if (int32_t r = open_sink(failure != nullptr, label, &sink, false, overflow)) return r;
    const bool narrow = (uint64_t)out->count < 0xFFFFFFFFull && (uint64_t)g.total < 0xFFFFFFFFull;
    const int32_t st = narrow ? run_scatter<uint32_t>(mode, target, indices, updates, out, g, sink)
                              : run_scatter<uint64_t>(mode, target, indices, updates, out, g, sink);
    if (st) return st;
    return close_sink(sink, label, failure, false, overflow);
}

int32_t scatter_operands(const char *what, const chelis_gpu_tensor *target, const chelis_gpu_tensor *indices,
                         const chelis_gpu_tensor *updates, const chelis_gpu_tensor *out) {
    if (int32_t s = check_tensor(target, "target")) return s;
    if (int32_t s = check_tensor(indices, "indices")) return s;
    if (int32_t s = check_tensor(updates, "updates")) return s;
    if (int32_t s = check_out(out, what)) return s;
    if (indices->dtype != CHELIS_DTYPE_I32 && indices->dtype != CHELIS_DTYPE_I64)
        return set_error(CHELIS_HIP_EDOMAIN, "%s: indices must be i32 or i64", what);
    if (out->dtype != target->dtype || updates->dtype != target->dtype)
        return set_error(CHELIS_HIP_EDOMAIN, "%s: target, updates and output need one dtype", what);
    if (out->rank != target->rank || target->rank > 8)
        return set_error(CHELIS_HIP_EDOMAIN, "%s: the output has the target's shape (rank <= 8)", what);
    for (int32_t a = 0; a < target->rank; ++a)
        if (out->shape[a] != target->shape[a])
            return set_error(CHELIS_HIP_EDOMAIN, "%s: the output has the target's shape", what);
    return CHELIS_HIP_OK;
}
}  // namespace

extern "C" int32_t chelis_hip_scatter(int32_t add, const chelis_gpu_tensor *target, const chelis_gpu_tensor *indices,
                                      const chelis_gpu_tensor *updates, int32_t axis, int32_t batch_rank,
                                      const chelis_gpu_tensor *out, chelis_hip_numeric_failure *failure) {
    const char *what = add ? "scatter" : "scatter_replace";
    if (int32_t s = scatter_operands(what, target, indices, updates, out)) return s;
    if (axis < 0 || axis >= target->rank || batch_rank < 0 || batch_rank > axis || batch_rank > indices->rank)
        return set_error(CHELIS_HIP_EDOMAIN, "%s: axis %d / batch_rank %d outside the operands", what, axis,
                         batch_rank);
    // emit.rs:3993-4042: the updates have the gathered shape, paired batch
    // extents agree; either failing is the domain trap
    const std::string trap = std::string("numeric trap: domain in ") + what + " at i64";
    bool shape_ok = updates->rank == target->rank - 1 + indices->rank - batch_rank;
    for (int32_t a = 0, k = 0; shape_ok && a < target->rank; ++a) {
        if (a == axis) {
            for (int32_t q = batch_rank; q < indices->rank && shape_ok; ++q)
                shape_ok = updates->shape[k++] == indices->shape[q];
        } else {
            shape_ok = updates->shape[k++] == target->shape[a];
        }
    }
    int64_t batch = 1, before = 1, after = 1;
    for (int32_t a = 0; a < batch_rank; ++a) {
        shape_ok = shape_ok && target->shape[a] == indices->shape[a];
        batch *= target->shape[a];
    }
    if (!shape_ok) return set_error(CHELIS_HIP_EDOMAIN, "%s", trap.c_str());
    for (int32_t a = 0; a < axis; ++a) before *= target->shape[a];
    for (int32_t a = axis + 1; a < target->rank; ++a) after *= target->shape[a];
    ScatterGeom g{};
    g.axis_size = target->shape[axis];
    g.after = after;
    g.index_count = batch == 0 ? 0 : indices->count / batch;
    g.outer_per_batch = (batch == 0 || before == 0) ? 1 : before / batch;
    g.total = updates->count;
    if (g.total && (g.after == 0 || g.index_count == 0)) g.total = 0;
    return scatter_common(add ? 1 : 0, target, indices, updates, out, g, failure);
}

extern "C" int32_t chelis_hip_scatter_elements(const chelis_gpu_tensor *data, const chelis_gpu_tensor *indices,
                                               const chelis_gpu_tensor *updates, int32_t axis,
                                               const chelis_gpu_tensor *out, chelis_hip_numeric_failure *failure) {
    if (int32_t s = scatter_operands("scatter_elements", data, indices, updates, out)) return s;
    if (axis < 0 || axis >= data->rank)
        return set_error(CHELIS_HIP_EDOMAIN, "scatter_elements: axis %d outside the operands", axis);
    // emit.rs:4160-4168: the updates have the indices' shape, every operand
    // the data's rank (crates/chelis-abi/src/metadata.rs:831-846: off the axis no index
    // extent passes the data's)
    bool shape_ok = indices->rank == data->rank && updates->rank == data->rank;
    for (int32_t a = 0; shape_ok && a < data->rank; ++a)
        shape_ok = updates->shape[a] == indices->shape[a] && (a == axis || indices->shape[a] <= data->shape[a]);
    if (!shape_ok) return set_error(CHELIS_HIP_EDOMAIN, "numeric trap: domain in scatter_elements at i64");
    ScatterGeom g{};
    g.elements = 1;
    g.rank = data->rank;
    g.axis = axis;
    g.total = updates->count;
    for (int32_t a = 0; a < data->rank; ++a) {
        g.idx_shape[a] = indices->shape[a];
        g.target_shape[a] = data->shape[a];
    }
    return scatter_common(2, data, indices, updates, out, g, failure);
}

extern "C" int32_t chelis_hip_take_numeric_failure(chelis_hip_numeric_failure *failure) {
    if (!failure) return set_error(CHELIS_HIP_EDOMAIN, "take_numeric_failure: null record");
    int32_t *words = status_words(nullptr);
    if (!words) return set_error(CHELIS_HIP_EHIP, "no HIP device status words");
    CHELIS_HIP_TRY(hipStreamSynchronize(stream()));
    unsigned long long word = 0ull;
    if (int32_t s = take_word(reinterpret_cast<unsigned long long *>(words + 2), &word)) return s;
    int device = 0;
    CHELIS_HIP_TRY(hipGetDevice(&device));
    Label label;
    {
        std::lock_guard<std::mutex> lock(g_fail_mutex);
        std::vector<Label> &labels = g_labels[device];
        const uint64_t seq = word ? (~word) >> kSeqShift : 0;
        if (word && seq < labels.size()) label = labels[seq];
        labels.clear();
    }
    return fill_failure(failure, word, label, reinterpret_cast<const long long *>(words + 6));
}

}  // namespace chelis

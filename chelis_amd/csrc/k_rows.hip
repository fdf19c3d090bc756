// Row regions on gfx950: softmax, causal scaled softmax, softmax adjoint and
// layer norm over the last axis, each as ONE kernel that reads its row once
// from HBM into registers and writes its result once.
//
// Layout of a row in registers. A row of n elements is treated as the
// power-of-two capacity CAP = S * 64W * V >= n, padded past n. The row is
// cut into S segments of 64W*V elements; in segment s, thread t holds the
// V consecutive elements starting at s*64W*V + t*V, loaded with one 16-byte
// vector load, so each load instruction of a wave covers one contiguous
// 1 KiB span (fully coalesced).
//
// Canonical sum tree ([05-OP-30]). Every (segment, thread) block is an
// aligned power-of-two run of leaves, so the adjacent-pair tree over the
// padded row is: an in-register tree over the V leaves, then a wave64
// butterfly (xor 1,2,...,32: step m joins the aligned blocks of 2^m
// threads), then a tree over the W waves through LDS, then a tree over the
// S segments. Padding leaves are -0.0, the exact additive identity
// (x + -0 = x for every x under round-to-nearest), and a power-of-two tree
// over the padded row has the same value as the adjacent-pair tree with an
// odd carry over the n real leaves. IEEE addition is commutative, so both
// butterfly partners hold the same bits.
//
// max_reduce ([05-OP-12]) combines with max_first in index order: in-lane
// left to right, butterfly with the lower lane as the left operand,
// waves and segments in order. Padding is -inf, which never displaces an
// earlier element.
#include "chain.h"

#include <initializer_list>

namespace chelis {
namespace {

// 16-byte native vectors (the nontemporal builtins take clang vector types).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
template <typename T, int V>
struct VecT;
template <>
struct VecT<float, 4> {
    using type = f32x4;
};
template <>
struct VecT<double, 2> {
    using type = f64x2;
};

// Streaming rows are read once and written once: NT selects the
// nontemporal (streaming) cache policy for them; vectors shared by every row
// (layer norm's gamma and beta) use the default policy.
template <bool NT, typename Q>
__device__ inline Q vload(const Q *p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT, typename Q>
__device__ inline void vstore(Q v, Q *p) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

template <typename T>
__device__ inline T neg_inf() {
    return -__builtin_huge_val();
}
template <>
__device__ inline float neg_inf<float>() {
    return -__builtin_huge_valf();
}

template <typename T>
__device__ inline T exp_leaf(T v);
template <>
__device__ inline float exp_leaf<float>(float v) {
    return expf_cr(v);
}
template <>
__device__ inline double exp_leaf<double>(double v) {
    return leaf_exp<double>(v);
}

// 2^(j/64), j = 0..63, held one entry per lane (lane j holds T[j]); a
// lookup is a wave64 shuffle, so every lane of the wave must be active.
struct ExpTableLanes {
    double t;
    __device__ explicit ExpTableLanes(int lane) : t(chelis_exp2_64_tab[lane][0]) {}
    __device__ double operator()(int j) const { return __shfl(t, j, 64); }
};

// 2^(j/64) as a double-double, read from the block's LDS copy: one 16-byte
// LDS read per lookup where a lane-held copy took four lane shuffles and
// four registers (the f64 softmax row: 58 against 64-68 us for [4096, 4096]
// on one box, bit-identical).
struct Exp2TableLds {
    const double2 *t;
    __device__ void operator()(int j, double &h, double &l) const {
        const double2 e = t[j];
        h = e.x;
        l = e.y;
    }
    // the high part alone (the faithful exp)
    __device__ double operator()(int j) const { return t[j].x; }
};

// The exp table of each dtype, built before the row loads so waiting for it
// never waits for a row: binary32 holds it one entry per lane, binary64 in
// LDS (filled by the kernel's first wave).
template <typename T>
struct RowExpTab;
template <>
struct RowExpTab<float> {
    using type = ExpTableLanes;
    __device__ static type make(int lane, const double2 *) { return type(lane); }
};
template <>
struct RowExpTab<double> {
    using type = Exp2TableLds;
    __device__ static type make(int, const double2 *lds) { return type{lds}; }
};

// Which of a lane's NE exp results need the correctly rounded fallback.
// Up to 16 per lane: one wave-uniform lane mask per element (scalar
// registers, set straight from the compare); beyond that: a per-lane bit set.
template <int NE, bool UNIFORM = (NE <= 16)>
struct SlowSet;
template <int NE>
struct SlowSet<NE, true> {
    uint64_t lanes[NE];
    uint64_t all = 0;
    __device__ void set(int k, bool slow) {
        lanes[k] = __ballot(slow);
        all |= lanes[k];
    }
    __device__ bool any() const { return all != 0; }
    __device__ bool has(int k, int lane) const { return (lanes[k] >> lane) & 1u; }
};
template <int NE>
struct SlowSet<NE, false> {
    static_assert(NE <= 64, "one bit per element");
    uint64_t bits = 0;
    __device__ void set(int k, bool slow) { bits |= (uint64_t)slow << k; }
    __device__ bool any() const { return __any(bits != 0); }
    __device__ bool has(int k, int) const { return (bits >> k) & 1u; }
};

// The rare correctly rounded fallback stays out of line: inlined 16 times it
// would dominate the kernel's code.
__device__ __noinline__ float expf_slow(float x) { return expf_cr_dd(x); }

// Per-row geometry: which row this wave group owns and where it starts.
template <int W, int R>
struct RowCoord {
    int lane, wave_in_row, row_in_block, tid_in_row;
    int64_t row;
    __device__ RowCoord() {
        const int tid = threadIdx.x;
        lane = tid & 63;
        const int wave = tid >> 6;
        wave_in_row = wave % W;
        row_in_block = wave / W;
        tid_in_row = wave_in_row * 64 + lane;
        row = (int64_t)blockIdx.x * R + row_in_block;
    }
};

template <typename T, int V, int S, int W, bool NT = true>
__device__ inline void load_row(const T *__restrict__ p, int64_t n, bool vec_ok, int tid_in_row, T pad,
                                T (&v)[S][V]) {
    constexpr int SEG = 64 * W * V;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int64_t base = (int64_t)s * SEG + (int64_t)tid_in_row * V;
        if (vec_ok && base + V <= n) {
            typename VecT<T, V>::type q = vload<NT>(reinterpret_cast<const typename VecT<T, V>::type *>(p + base));
            const T *qe = reinterpret_cast<const T *>(&q);
#pragma unroll
            for (int i = 0; i < V; ++i) v[s][i] = qe[i];
        } else {
#pragma unroll
            for (int i = 0; i < V; ++i) v[s][i] = (base + i < n) ? p[base + i] : pad;
        }
    }
}

template <typename T, int V, int S, int W>
__device__ inline void store_row(T *__restrict__ p, int64_t n, bool vec_ok, int tid_in_row, const T (&v)[S][V]) {
    constexpr int SEG = 64 * W * V;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int64_t base = (int64_t)s * SEG + (int64_t)tid_in_row * V;
        if (vec_ok && base + V <= n) {
            typename VecT<T, V>::type q;
            T *qe = reinterpret_cast<T *>(&q);
#pragma unroll
            for (int i = 0; i < V; ++i) qe[i] = v[s][i];
            vstore<true>(q, reinterpret_cast<typename VecT<T, V>::type *>(p + base));
        } else {
#pragma unroll
            for (int i = 0; i < V; ++i)
                if (base + i < n) p[base + i] = v[s][i];
        }
    }
}

// Canonical tree over the padded row; every thread of the row gets the total.
template <typename T, int V, int S, int W, int R>
__device__ inline T row_tree_sum(const T (&v)[S][V], T *lds, const RowCoord<W, R> &c) {
    T seg[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        T a[V];
#pragma unroll
        for (int i = 0; i < V; ++i) a[i] = v[s][i];
#pragma unroll
        for (int w = V; w > 1; w >>= 1)
#pragma unroll
            for (int i = 0; i < w / 2; ++i) a[i] = a[2 * i] + a[2 * i + 1];
        seg[s] = wave_tree_sum(a[0]);
    }
    if constexpr (W > 1) {
        if (c.lane == 0)
#pragma unroll
            for (int s = 0; s < S; ++s) lds[(c.row_in_block * W + c.wave_in_row) * S + s] = seg[s];
        __syncthreads();
#pragma unroll
        for (int s = 0; s < S; ++s) {
            T p[W];
#pragma unroll
            for (int w = 0; w < W; ++w) p[w] = lds[(c.row_in_block * W + w) * S + s];
#pragma unroll
            for (int w = W; w > 1; w >>= 1)
#pragma unroll
                for (int i = 0; i < w / 2; ++i) p[i] = p[2 * i] + p[2 * i + 1];
            seg[s] = p[0];
        }
        __syncthreads();
    }
#pragma unroll
    for (int w = S; w > 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w / 2; ++i) seg[i] = seg[2 * i] + seg[2 * i + 1];
    return seg[0];
}

// Plain IEEE maximum over the padded row (v_max: a NaN operand yields the
// other one, and +0/-0 ties are unordered). Softmax uses it in place of
// [05-OP-12]'s first-NaN / first-representation rule because the two give
// identical softmax bits: a NaN anywhere in the row makes that element's
// x - m NaN, hence the tree sum NaN and every output the canonical NaN under
// either rule; and a zero maximum enters only through x - m, where
// x - (+0) and x - (-0) differ at most in the sign of a zero, which exp maps
// to the same 1.
template <typename T, int V, int S, int W, int R>
__device__ inline T row_max_plain(const T (&v)[S][V], T *lds, const RowCoord<W, R> &c) {
    T x = v[0][0];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < V; ++i) x = vmax(x, v[s][i]);
    x = wave_vmax(x);
    if constexpr (W > 1) {
        if (c.lane == 0) lds[c.row_in_block * W + c.wave_in_row] = x;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < W; ++w) x = vmax(x, lds[c.row_in_block * W + w]);
        __syncthreads();
    }
    return x;
}

// v / total at the dtype. binary32: the quotient is formed as
// (double)v * (1 / (double)total) and rounded once to binary32. That is the
// correctly rounded v / total: the exact quotient of two binary32 values is
// never closer than 2^-49 relative to a binary32 rounding midpoint (it is
// X 2^a / (T 2^b) with 24-bit X, T against a midpoint M 2^c with 25-bit M,
// and X 2^a - T M 2^(b+c) is a nonzero multiple of 2^min(a, b+c); the
// subnormal range keeps an absolute gap of at least 2^-150 / T), while the
// binary64 product is within 2^-52 relative of it.
template <typename T>
struct RowDiv {
    T total;
    double inv;
    __device__ explicit RowDiv(T t) : total(t), inv(1.0 / (double)t) {}
    __device__ T operator()(T v) const { return canon(quot_f32(v, inv)); }
};

__device__ __noinline__ double div_full(double v, double t) { return v / t; }

// binary64: the steps of the device's IEEE division (v_div_scale_f64 of
// both operands, v_rcp_f64 with two Newton steps, product, residual, fma,
// v_div_fixup_f64), with the reciprocal - which depends only on the
// divisor - formed once per row. The steps are taken as they are where the
// scale steps are the identity: a divisor in [1, 2^20] (the row totals)
// and a dividend that is 0 or at least 2^-960 (v_div_scale_f64 scales a
// dividend whose biased exponent is at most 53, or whose quotient would be
// subnormal); any other element takes the full division.
template <>
struct RowDiv<double> {
    double total, rcp;
    bool fast;
    __device__ explicit RowDiv(double t) : total(t), fast(t >= 1.0 && t <= 0x1p20) {
        double r = __builtin_amdgcn_rcp(t);
        double e = fma(-t, r, 1.0);
        r = fma(r, e, r);
        e = fma(-t, r, 1.0);
        rcp = fma(r, e, r);
    }
    __device__ double operator()(double v) const {
        if (fast && (v == 0.0 || v >= 0x1p-960)) {
            const double q = v * rcp;
            const double r = fma(-total, q, v);
            return canon(__builtin_amdgcn_div_fixup(fma(r, rcp, q), total, v));
        }
        return canon(div_full(v, total));
    }
};

// The value softmax takes x - max of: element j of a row, optionally
// as where(j <= qi, x * scale, -inf) (masked 1: causal, masked 2: scale only).
template <typename T>
__device__ inline T softmax_arg(T raw, int64_t j, int64_t qi, int masked, T scale) {
    if (!masked) return raw;
    const T sc = canon(raw * scale);
    return (masked == 2 || j <= qi) ? sc : neg_inf<T>();
}

// One row: v holds the raw row (padding -inf) on entry and the softmax on
// exit; xr is the row in memory (re-read only by the rare exp fallback).
// FAITHFUL (binary64 only): the faithful exp and one reciprocal per row in
// place of the correctly rounded exp and the IEEE division.
template <typename T, int V, int S, int W, int R, bool FAITHFUL = false>
__device__ inline void softmax_row(T (&v)[S][V], const T *__restrict__ xr, int64_t row, int64_t n, int masked,
                                   T scale, int64_t q_len, T *lds, const RowCoord<W, R> &c,
                                   const typename RowExpTab<T>::type &tab) {
    constexpr int SEG = 64 * W * V;
    const int64_t qi = masked ? row % q_len : 0;
    if (masked) {
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const int64_t j = (int64_t)s * SEG + (int64_t)c.tid_in_row * V + i;
                if (j < n) v[s][i] = softmax_arg(v[s][i], j, qi, masked, scale);
            }
    }
    const T m = row_max_plain<T, V, S, W, R>(v, lds, c);
    const bool full = n == (int64_t)S * SEG;
    if constexpr (sizeof(T) == 4) {
        // exp(x - m) in place: the branch-free fast path for every element
        // (2^(j/64) from the lane-held table), then one wave-uniform pass of
        // the correctly rounded core over the few flagged elements, whose
        // argument is formed again from the row in memory. x - m is <= 0 or
        // NaN (m is the row maximum), so the NONPOS path applies.
        SlowSet<S * V> flagged;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < V; ++i) {
                bool slow;
                v[s][i] = expf_fast<true>(v[s][i] - m, tab, slow);
                flagged.set(s * V + i, slow);
            }
        if (flagged.any()) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    const int64_t j = (int64_t)s * SEG + (int64_t)c.tid_in_row * V + i;
                    if (flagged.has(s * V + i, c.lane) && (full || j < n))
                        v[s][i] = expf_slow(softmax_arg(xr[j], j, qi, masked, scale) - m);
                }
        }
        if (!full) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    const int64_t j = (int64_t)s * SEG + (int64_t)c.tid_in_row * V + i;
                    if (j >= n) v[s][i] = T(-0.0);
                }
        }
        const T total = row_tree_sum<T, V, S, W, R>(v, lds, c);
        if (total != total) {
            // a NaN total makes every quotient the canonical NaN
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) v[s][i] = canon(total);
        } else {
            // total >= 1 (the maximum contributes exp(0)) or +inf: finite
            // e / total needs no NaN finalization
            const double inv = 1.0 / (double)total;
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) v[s][i] = quot_f32(v[s][i], inv);
        }
    } else if constexpr (FAITHFUL) {
        // the default binary64 row: exp(x - m) faithful (within 1 ulp, no
        // fallback pass), the canonical tree total, then e * (1 / total):
        // within a few ulps of the correctly rounded quotients. A NaN
        // argument yields a NaN exp, hence a NaN total and every output the
        // canonical NaN, as in the exact row.
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < V; ++i) v[s][i] = exp_nonpos_faithful(v[s][i] - m, tab);
        if (!full) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    const int64_t j = (int64_t)s * SEG + (int64_t)c.tid_in_row * V + i;
                    if (j >= n) v[s][i] = T(-0.0);
                }
        }
        const T total = row_tree_sum<T, V, S, W, R>(v, lds, c);
        if (total != total) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) v[s][i] = canon(total);
        } else {
            // 1 <= total <= n: every product is finite
            const T inv = T(1) / total;
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) v[s][i] = v[s][i] * inv;
        }
    } else {
        // exp(x - m) in place, as for binary32: the binary64 fast path for
        // every element (2^(j/64) as a double-double from the lane-held
        // table), then one wave-uniform pass of the fixed-point path over the
        // flagged elements (about one in 2^19, and NaN arguments).
        SlowSet<S * V> flagged;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < V; ++i) {
                bool slow;
                v[s][i] = exp_fast<true>(v[s][i] - m, tab, slow);
                flagged.set(s * V + i, slow);
            }
        if (flagged.any()) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    const int64_t j = (int64_t)s * SEG + (int64_t)c.tid_in_row * V + i;
                    if (flagged.has(s * V + i, c.lane) && (full || j < n))
                        v[s][i] = exp_slow64(softmax_arg(xr[j], j, qi, masked, scale) - m);
                }
        }
        if (!full) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    const int64_t j = (int64_t)s * SEG + (int64_t)c.tid_in_row * V + i;
                    if (j >= n) v[s][i] = T(-0.0);
                }
        }
        const RowDiv<T> div(canon(row_tree_sum<T, V, S, W, R>(v, lds, c)));
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < V; ++i) v[s][i] = div(v[s][i]);
    }
}

// softmax over the last axis, optionally of where(j <= i, x * scale, -inf)
// (causal != 0, q_len = rows per score matrix). DENSE instances serve the
// common case (no mask, row length equal to the register capacity S*64W*V,
// 16-byte aligned rows) with every bound test folded away. FAITHFUL as for
// softmax_row.
template <typename T, int V, int S, int W, int R, bool DENSE, bool FAITHFUL = false>
__global__ __launch_bounds__(64 * W * R) void softmax_kernel(const T *__restrict__ x, T *__restrict__ y,
                                                              int64_t rows, int64_t n_arg, int64_t ldx, int64_t ldy,
                                                              bool vec_ok_arg, int masked_arg, T scale,
                                                              int64_t q_len) {
    __shared__ T lds[R * W * S];
    constexpr int SEG = 64 * W * V;
    const int64_t n = DENSE ? (int64_t)S * SEG : n_arg;
    const bool vec_ok = DENSE || vec_ok_arg;
    const int masked = DENSE ? 0 : masked_arg;
    __shared__ double2 exp_tab[sizeof(T) == 8 ? 64 : 1];
    if constexpr (sizeof(T) == 8) {
        if (threadIdx.x < 64) exp_tab[threadIdx.x] = double2{chelis_exp2_64_tab[threadIdx.x][0], chelis_exp2_64_tab[threadIdx.x][1]};
        __syncthreads();
    }
    RowCoord<W, R> c;
    if (c.row >= rows) return;  // whole row groups exit together (R rows per block, W waves each)
    const T *xr = x + c.row * ldx;
    const typename RowExpTab<T>::type tab = RowExpTab<T>::make(c.lane, exp_tab);
    T v[S][V];
    // causal rows read only j <= qi: the mask turns every later element into
    // -inf whatever it holds, which is the padding value
    const int64_t n_load = masked == 1 ? (c.row % q_len + 1 < n ? c.row % q_len + 1 : n) : n;
    load_row<T, V, S, W>(xr, n_load, vec_ok, c.tid_in_row, neg_inf<T>(), v);
    softmax_row<T, V, S, W, R, FAITHFUL>(v, xr, c.row, n, masked, scale, q_len, lds, c, tab);
    store_row<T, V, S, W>(y + c.row * ldy, n, vec_ok, c.tid_in_row, v);
}

// dx = y * (g - sum(g * y)) over the last axis.
template <typename T, int V, int S, int W, int R>
__global__ __launch_bounds__(64 * W * R) void softmax_adjoint_kernel(const T *__restrict__ y,
                                                                      const T *__restrict__ g, T *__restrict__ dx,
                                                                      int64_t rows, int64_t n, int64_t ldy,
                                                                      int64_t ldg, int64_t ldd, bool vec_ok) {
    __shared__ T lds[R * W * S];
    RowCoord<W, R> c;
    if (c.row >= rows) return;
    T yv[S][V], gv[S][V], t[S][V];
    load_row<T, V, S, W>(y + c.row * ldy, n, vec_ok, c.tid_in_row, T(-0.0), yv);
    load_row<T, V, S, W>(g + c.row * ldg, n, vec_ok, c.tid_in_row, T(-0.0), gv);
    constexpr int SEG = 64 * W * V;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const int64_t j = (int64_t)s * SEG + (int64_t)c.tid_in_row * V + i;
            t[s][i] = (j < n) ? canon(gv[s][i] * yv[s][i]) : T(-0.0);
        }
    const T total = canon(row_tree_sum<T, V, S, W, R>(t, lds, c));
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < V; ++i) t[s][i] = canon(yv[s][i] * canon(gv[s][i] - total));
    store_row<T, V, S, W>(dx + c.row * ldd, n, vec_ok, c.tid_in_row, t);
}

// layer_norm: mean = tree(x)/n; c = x - mean; var = tree(c*c)/n;
// y = (c / sqrt(var + eps)) * gamma + beta, every primitive finalized.
template <typename T, int V, int S, int W, int R>
__global__ __launch_bounds__(64 * W * R) void layer_norm_kernel(const T *__restrict__ x, const T *__restrict__ gamma,
                                                                 const T *__restrict__ beta, T *__restrict__ y,
                                                                 int64_t rows, int64_t n, int64_t ldx, int64_t ldy,
                                                                 bool vec_ok, T eps) {
    __shared__ T lds[R * W * S];
    RowCoord<W, R> c;
    if (c.row >= rows) return;
    T v[S][V], q[S][V], gm[S][V], bt[S][V];
    load_row<T, V, S, W>(x + c.row * ldx, n, vec_ok, c.tid_in_row, T(-0.0), v);
    // gamma/beta are [n] vectors shared by every row: their loads go out with
    // the row's, ahead of the reductions' barriers (after them each row waited
    // out two more cache round trips: [65536,1024] 90.8 -> 88.5 us)
    load_row<T, V, S, W, false>(gamma, n, vec_ok, c.tid_in_row, T(0), gm);
    load_row<T, V, S, W, false>(beta, n, vec_ok, c.tid_in_row, T(0), bt);
    const T extent = (T)n;
    const T mean = canon(canon(row_tree_sum<T, V, S, W, R>(v, lds, c)) / extent);
    constexpr int SEG = 64 * W * V;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const int64_t j = (int64_t)s * SEG + (int64_t)c.tid_in_row * V + i;
            v[s][i] = canon(v[s][i] - mean);
            q[s][i] = (j < n) ? canon(v[s][i] * v[s][i]) : T(-0.0);
        }
    const T var = canon(canon(row_tree_sum<T, V, S, W, R>(q, lds, c)) / extent);
    const T denom = canon_bits(sqrt(canon(var + eps)));
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < V; ++i) v[s][i] = canon(canon(v[s][i] / denom) * gm[s][i]);
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < V; ++i) v[s][i] = canon(v[s][i] + bt[s][i]);
    store_row<T, V, S, W>(y + c.row * ldy, n, vec_ok, c.tid_in_row, v);
}

// ---------------------------------------------------------------- dispatch
// Instantiated shapes: (S, W, R) per capacity. V is 16 bytes of T.
enum class RowOp { Softmax, SoftmaxAdjoint, LayerNorm };

struct RowArgs {
    const void *a, *b, *c;
    void *out;
    int64_t rows, n, lda, ldb, ldo;
    bool vec_ok;
    int masked;
    double scale;
    int64_t q_len;
    double eps;
};

template <typename T, int V, int S, int W, int R>
int32_t launch_shape(RowOp op, const RowArgs &a, hipStream_t st) {
    const unsigned grid = grid_for(a.rows, R);
    if (!grid_fits(grid, 64 * W * R)) return set_error(CHELIS_HIP_EUNSUPPORTED, "rows: %lld rows exceed one launch",
                                                       (long long)a.rows);
    const dim3 block(64 * W * R);
    switch (op) {
        case RowOp::Softmax: {
            const bool dense = !a.masked && a.vec_ok && a.n == (int64_t)S * 64 * W * V;
            // binary64 outside the exact mode: the faithful row
            if constexpr (sizeof(T) == 8) {
                if (!exact_mode()) {
                    if (dense)
                        softmax_kernel<T, V, S, W, R, true, true><<<grid, block, 0, st>>>(
                            (const T *)a.a, (T *)a.out, a.rows, a.n, a.lda, a.ldo, a.vec_ok, a.masked, (T)a.scale,
                            a.q_len);
                    else
                        softmax_kernel<T, V, S, W, R, false, true><<<grid, block, 0, st>>>(
                            (const T *)a.a, (T *)a.out, a.rows, a.n, a.lda, a.ldo, a.vec_ok, a.masked, (T)a.scale,
                            a.q_len);
                    break;
                }
            }
            if (dense) {
                softmax_kernel<T, V, S, W, R, true><<<grid, block, 0, st>>>(
                    (const T *)a.a, (T *)a.out, a.rows, a.n, a.lda, a.ldo, a.vec_ok, a.masked, (T)a.scale, a.q_len);
            } else {
                softmax_kernel<T, V, S, W, R, false><<<grid, block, 0, st>>>(
                    (const T *)a.a, (T *)a.out, a.rows, a.n, a.lda, a.ldo, a.vec_ok, a.masked, (T)a.scale, a.q_len);
            }
            break;
        }
        case RowOp::SoftmaxAdjoint:
            softmax_adjoint_kernel<T, V, S, W, R><<<grid, block, 0, st>>>(
                (const T *)a.a, (const T *)a.b, (T *)a.out, a.rows, a.n, a.lda, a.ldb, a.ldo, a.vec_ok);
            break;
        case RowOp::LayerNorm:
            layer_norm_kernel<T, V, S, W, R><<<grid, block, 0, st>>>(
                (const T *)a.a, (const T *)a.b, (const T *)a.c, (T *)a.out, a.rows, a.n, a.lda, a.ldo, a.vec_ok,
                (T)a.eps);
            break;
    }
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

// Capacity ladder: CAP = S * 64W * V, smallest power of two >= n.
template <typename T>
int32_t launch_rows(RowOp op, const RowArgs &a) {
    constexpr int V = 16 / sizeof(T);
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    const int64_t seg1 = 64 * V;  // one wave, one segment
    const int64_t n = a.n;
    if (n <= seg1) return launch_shape<T, V, 1, 1, 4>(op, a, st);
    if (n <= 2 * seg1) return launch_shape<T, V, 2, 1, 4>(op, a, st);
    // binary32 rows of 513-1024: two waves per row, two segments each
    // (23.4 against 24.2 us for [16384, 1024] with one wave of four
    // segments, same box: the shorter per-wave dependency chain keeps more
    // stores in flight); other rows of this bucket: one row per 64-lane
    // block, so blocks retire independently and the waves of a CU drift
    // apart, one wave's loads overlapping another's arithmetic
    if (n <= 4 * seg1) {
        if constexpr (sizeof(T) == 4) return launch_shape<T, V, 2, 2, 1>(op, a, st);
        return launch_shape<T, V, 4, 1, 1>(op, a, st);
    }
    if (n <= 8 * seg1) return launch_shape<T, V, 8, 1, 2>(op, a, st);
    if (n <= 16 * seg1) return launch_shape<T, V, 4, 4, 1>(op, a, st);
    if (n <= 32 * seg1) return launch_shape<T, V, 8, 4, 1>(op, a, st);
    if (n <= 64 * seg1) return launch_shape<T, V, 8, 8, 1>(op, a, st);
    if (n <= 128 * seg1) return launch_shape<T, V, 8, 16, 1>(op, a, st);
    if (n <= 256 * seg1) return launch_shape<T, V, 16, 16, 1>(op, a, st);
    return set_error(CHELIS_HIP_EUNSUPPORTED, "row length %lld exceeds the in-register row capacity %lld",
                     (long long)n, (long long)(256 * seg1));
}

int32_t dispatch(chelis_dtype dt, RowOp op, const RowArgs &a) {
    if (a.rows == 0 || a.n == 0) return CHELIS_HIP_OK;
    return dt == CHELIS_DTYPE_F32 ? launch_rows<float>(op, a) : launch_rows<double>(op, a);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int32_t check_rows_pair(const chelis_gpu_tensor *x, const chelis_gpu_tensor *y, RowView *vx, RowView *vy,
                        const char *what) {
    int32_t s;
    if ((s = check_tensor(x, "x")) || (s = check_tensor(y, "y"))) return s;
    if (!is_float(x->dtype) || x->dtype != y->dtype)
        return set_error(CHELIS_HIP_EDOMAIN, "%s: x and y must share an f32 or f64 dtype", what);
    if (!same_shape(x, y)) return set_error(CHELIS_HIP_EDOMAIN, "%s: x and y shapes differ", what);
    if (!row_view(x, vx) || !row_view(y, vy))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "%s: last axis must be contiguous with uniform row stride", what);
    return CHELIS_HIP_OK;
}

// ---------------------------------------------------------------- long rows
// Rows longer than the register capacity (64 * 256 * 16 / sizeof(T): 65 536
// binary32 or 32 768 binary64 values) run as the graph the region stands
// for, one launch per reduction and per elementwise pass, in the same
// primitive order as the row kernels: the reductions take the canonical
// tree over the whole row (aligned segment totals joined pass by pass), the
// chains finalize every primitive, so the results are bit-identical to what
// the row kernels would give (and to the C lane's).
constexpr int64_t kRowCapacityBytes = 64 * 256 * 16;

struct Rows2 {
    int64_t shape[2], strides[2];
    chelis_gpu_tensor t{};
    Rows2(void *data, chelis_dtype dt, int64_t rows, int64_t n, int64_t s_row, int64_t s_col, int64_t cap) {
        shape[0] = rows, shape[1] = n, strides[0] = s_row, strides[1] = s_col;
        t.data = data;
        t.dtype = dt;
        t.rank = 2;
        t.shape = shape;
        t.strides = strides;
        t.count = rows * n;
        t.byte_capacity = cap;
    }
};
struct Vec1 {
    int64_t shape[1], strides[1];
    chelis_gpu_tensor t{};
    Vec1(void *data, chelis_dtype dt, int64_t n) {
        shape[0] = n, strides[0] = 1;
        t.data = data;
        t.dtype = dt;
        t.rank = 1;
        t.shape = shape;
        t.strides = strides;
        t.count = n;
        t.byte_capacity = n * dtype_width(dt);
    }
};

chelis_fused_step fstep(int op, int32_t a0, int32_t a1 = 0, double imm = 0.0) {
    chelis_fused_step st{};
    st.op = (uint8_t)op;
    st.args[0] = a0;
    st.args[1] = a1;
    st.imm = imm;
    return st;
}
constexpr int32_t prv(int32_t k) { return -(k + 1); }
chelis_fused_chain fchain(std::initializer_list<chelis_fused_step> steps) {
    chelis_fused_chain c{};
    for (const chelis_fused_step &st : steps) c.steps[c.n_steps++] = st;
    return c;
}

// Per-row scratch vectors, released (stream-ordered) at scope exit.
struct RowScratch {
    void *p = nullptr;
    size_t bytes = 0;
    explicit RowScratch(size_t b) : p(scratch_alloc(b)), bytes(b) {}
    ~RowScratch() { scratch_free(p, bytes); }
};

int32_t long_softmax(const chelis_gpu_tensor *x, const chelis_gpu_tensor *y, const RowView &vx, const RowView &vy) {
    const chelis_dtype dt = x->dtype;
    const int64_t w = dtype_width(dt), R = vx.rows, n = vx.n;
    RowScratch m(R * w), sum(R * w);
    if (!m.p || !sum.p) return set_error(CHELIS_HIP_EHIP, "softmax: row scratch of %lld bytes", (long long)(2 * R * w));
    const Rows2 X(x->data, dt, R, n, vx.ld, 1, x->byte_capacity), Y(y->data, dt, R, n, vy.ld, 1, y->byte_capacity);
    const Vec1 M(m.p, dt, R), S(sum.p, dt, R);
    const Rows2 Mb(m.p, dt, R, n, 1, 0, R * w), Sb(sum.p, dt, R, n, 1, 0, R * w);
    // m = max over the row; s = tree(exp(x - m)); y = exp(x - m) / s
    const chelis_gpu_tensor *in1[1] = {&X.t};
    if (int32_t st = chelis_hip_reduce(CHELIS_REDUCE_MAX, nullptr, in1, 1, 1, &M.t)) return st;
    const chelis_fused_chain e = fchain({fstep(CHELIS_FUSED_SUB, 0, 1), fstep(CHELIS_FUSED_EXP, prv(0))});
    const chelis_gpu_tensor *in2[2] = {&X.t, &Mb.t};
    if (int32_t st = chelis_hip_reduce(CHELIS_REDUCE_SUM, &e, in2, 2, 1, &S.t)) return st;
    const chelis_fused_chain q = fchain(
        {fstep(CHELIS_FUSED_SUB, 0, 1), fstep(CHELIS_FUSED_EXP, prv(0)), fstep(CHELIS_FUSED_DIV, prv(1), 2)});
    const chelis_gpu_tensor *in3[3] = {&X.t, &Mb.t, &Sb.t};
    return chelis_hip_fused_elementwise(&q, in3, 3, &Y.t);
}

int32_t long_softmax_adjoint(const chelis_gpu_tensor *y, const chelis_gpu_tensor *g, const chelis_gpu_tensor *dx,
                             const RowView &vy, const RowView &vg, const RowView &vd) {
    const chelis_dtype dt = y->dtype;
    const int64_t w = dtype_width(dt), R = vy.rows, n = vy.n;
    RowScratch tot(R * w);
    if (!tot.p) return set_error(CHELIS_HIP_EHIP, "softmax_adjoint: row scratch of %lld bytes", (long long)(R * w));
    const Rows2 Yv(y->data, dt, R, n, vy.ld, 1, y->byte_capacity), G(g->data, dt, R, n, vg.ld, 1, g->byte_capacity),
        D(dx->data, dt, R, n, vd.ld, 1, dx->byte_capacity);
    const Vec1 T(tot.p, dt, R);
    const Rows2 Tb(tot.p, dt, R, n, 1, 0, R * w);
    // t = tree(g * y); dx = y * (g - t)
    const chelis_fused_chain gy = fchain({fstep(CHELIS_FUSED_MUL, 0, 1)});
    const chelis_gpu_tensor *in2[2] = {&G.t, &Yv.t};
    if (int32_t st = chelis_hip_reduce(CHELIS_REDUCE_SUM, &gy, in2, 2, 1, &T.t)) return st;
    const chelis_fused_chain d = fchain({fstep(CHELIS_FUSED_SUB, 1, 2), fstep(CHELIS_FUSED_MUL, 0, prv(0))});
    const chelis_gpu_tensor *in3[3] = {&Yv.t, &G.t, &Tb.t};
    return chelis_hip_fused_elementwise(&d, in3, 3, &D.t);
}

int32_t long_layer_norm(const chelis_gpu_tensor *x, const chelis_gpu_tensor *gamma, const chelis_gpu_tensor *beta,
                        double eps, const chelis_gpu_tensor *y, const RowView &vx, const RowView &vy) {
    const chelis_dtype dt = x->dtype;
    const int64_t w = dtype_width(dt), R = vx.rows, n = vx.n;
    RowScratch tmp(R * w), mean(R * w), den(R * w);
    if (!tmp.p || !mean.p || !den.p)
        return set_error(CHELIS_HIP_EHIP, "layer_norm: row scratch of %lld bytes", (long long)(3 * R * w));
    const Rows2 X(x->data, dt, R, n, vx.ld, 1, x->byte_capacity), Y(y->data, dt, R, n, vy.ld, 1, y->byte_capacity);
    const Vec1 Tv(tmp.p, dt, R), Mv(mean.p, dt, R), Dv(den.p, dt, R);
    const Rows2 Mb(mean.p, dt, R, n, 1, 0, R * w), Db(den.p, dt, R, n, 1, 0, R * w);
    const Rows2 Gb(gamma->data, dt, R, n, 0, 1, gamma->byte_capacity), Bb(beta->data, dt, R, n, 0, 1, beta->byte_capacity);
    const double extent = (double)n;
    // mean = tree(x) / n
    const chelis_gpu_tensor *in1[1] = {&X.t};
    if (int32_t st = chelis_hip_reduce(CHELIS_REDUCE_SUM, nullptr, in1, 1, 1, &Tv.t)) return st;
    const chelis_fused_chain by_n = fchain({fstep(CHELIS_FUSED_CONST, 0, 0, extent), fstep(CHELIS_FUSED_DIV, 0, prv(0))});
    const chelis_gpu_tensor *t1[1] = {&Tv.t};
    if (int32_t st = chelis_hip_fused_elementwise(&by_n, t1, 1, &Mv.t)) return st;
    // var = tree((x - mean)^2) / n; denom = sqrt(var + eps)
    const chelis_fused_chain sq = fchain({fstep(CHELIS_FUSED_SUB, 0, 1), fstep(CHELIS_FUSED_MUL, prv(0), prv(0))});
    const chelis_gpu_tensor *in2[2] = {&X.t, &Mb.t};
    if (int32_t st = chelis_hip_reduce(CHELIS_REDUCE_SUM, &sq, in2, 2, 1, &Tv.t)) return st;
    const chelis_fused_chain dn = fchain({fstep(CHELIS_FUSED_CONST, 0, 0, extent), fstep(CHELIS_FUSED_DIV, 0, prv(0)),
                                          fstep(CHELIS_FUSED_CONST, 0, 0, eps), fstep(CHELIS_FUSED_ADD, prv(1), prv(2)),
                                          fstep(CHELIS_FUSED_SQRT, prv(3))});
    if (int32_t st = chelis_hip_fused_elementwise(&dn, t1, 1, &Dv.t)) return st;
    // y = ((x - mean) / denom) * gamma + beta
    const chelis_fused_chain out = fchain({fstep(CHELIS_FUSED_SUB, 0, 1), fstep(CHELIS_FUSED_DIV, prv(0), 2),
                                           fstep(CHELIS_FUSED_MUL, prv(1), 3), fstep(CHELIS_FUSED_ADD, prv(2), 4)});
    const chelis_gpu_tensor *in5[5] = {&X.t, &Mb.t, &Db.t, &Gb.t, &Bb.t};
    return chelis_hip_fused_elementwise(&out, in5, 5, &Y.t);
}

bool long_rows(chelis_dtype dt, int64_t n) { return n > kRowCapacityBytes / dtype_width(dt); }

}  // namespace
}  // namespace chelis

using namespace chelis;

extern "C" int32_t chelis_hip_softmax(const chelis_gpu_tensor *x, const chelis_gpu_tensor *y) {
    RowView vx, vy;
    if (int32_t s = check_rows_pair(x, y, &vx, &vy, "softmax")) return s;
    if (vx.rows && long_rows(x->dtype, vx.n)) return long_softmax(x, y, vx, vy);
    const int64_t V = 16 / dtype_width(x->dtype);
    RowArgs a{x->data, nullptr, nullptr, y->data, vx.rows, vx.n, vx.ld, 0, vy.ld,
              aligned16(x->data) && aligned16(y->data) && vx.ld % V == 0 && vy.ld % V == 0, 0, 1.0, 1, 0.0};
    return dispatch(x->dtype, RowOp::Softmax, a);
}

extern "C" int32_t chelis_hip_scaled_masked_softmax(const chelis_gpu_tensor *x, double scale, int32_t causal,
                                                    const chelis_gpu_tensor *y) {
    RowView vx, vy;
    if (int32_t s = check_rows_pair(x, y, &vx, &vy, "scaled_masked_softmax")) return s;
    if (x->rank < 2) return set_error(CHELIS_HIP_EDOMAIN, "scaled_masked_softmax: scores need rank >= 2");
    const int64_t q_len = x->shape[x->rank - 2];
    if (causal && q_len != vx.n)
        return set_error(CHELIS_HIP_EDOMAIN, "scaled_masked_softmax: causal mask needs square score matrices");
    const int64_t V = 16 / dtype_width(x->dtype);
    RowArgs a{x->data, nullptr, nullptr, y->data, vx.rows, vx.n, vx.ld, 0, vy.ld,
              aligned16(x->data) && aligned16(y->data) && vx.ld % V == 0 && vy.ld % V == 0,
              causal ? 1 : 2, scale, q_len > 0 ? q_len : 1, 0.0};
    return dispatch(x->dtype, RowOp::Softmax, a);
}

extern "C" int32_t chelis_hip_softmax_adjoint(const chelis_gpu_tensor *y, const chelis_gpu_tensor *g,
                                              const chelis_gpu_tensor *dx) {
    RowView vy, vg, vd;
    if (int32_t s = check_rows_pair(y, dx, &vy, &vd, "softmax_adjoint")) return s;
    if (int32_t s = check_tensor(g, "g")) return s;
    if (g->dtype != y->dtype || !same_shape(g, y) || !row_view(g, &vg))
        return set_error(CHELIS_HIP_EDOMAIN, "softmax_adjoint: g must match y");
    if (vy.rows && long_rows(y->dtype, vy.n)) return long_softmax_adjoint(y, g, dx, vy, vg, vd);
    const int64_t V = 16 / dtype_width(y->dtype);
    RowArgs a{y->data, g->data, nullptr, dx->data, vy.rows, vy.n, vy.ld, vg.ld, vd.ld,
              aligned16(y->data) && aligned16(g->data) && aligned16(dx->data) && vy.ld % V == 0 &&
                  vg.ld % V == 0 && vd.ld % V == 0,
              0, 1.0, 1, 0.0};
    return dispatch(y->dtype, RowOp::SoftmaxAdjoint, a);
}

extern "C" int32_t chelis_hip_layer_norm(const chelis_gpu_tensor *x, const chelis_gpu_tensor *gamma,
                                         const chelis_gpu_tensor *beta, double epsilon,
                                         const chelis_gpu_tensor *y) {
    RowView vx, vy;
    if (int32_t s = check_rows_pair(x, y, &vx, &vy, "layer_norm")) return s;
    int32_t s;
    if ((s = check_tensor(gamma, "gamma")) || (s = check_tensor(beta, "beta"))) return s;
    for (const chelis_gpu_tensor *p : {gamma, beta})
        if (p->dtype != x->dtype || p->rank != 1 || p->shape[0] != vx.n || (vx.n > 1 && p->strides[0] != 1))
            return set_error(CHELIS_HIP_EDOMAIN, "layer_norm: gamma/beta must be contiguous [hidden]");
    if (vx.n == 0) return set_error(CHELIS_HIP_EDOMAIN, "layer_norm: hidden extent must be positive");
    if (vx.rows && long_rows(x->dtype, vx.n)) return long_layer_norm(x, gamma, beta, epsilon, y, vx, vy);
    const int64_t V = 16 / dtype_width(x->dtype);
    RowArgs a{x->data, gamma->data, beta->data, y->data, vx.rows, vx.n, vx.ld, 0, vy.ld,
              aligned16(x->data) && aligned16(y->data) && aligned16(gamma->data) && aligned16(beta->data) &&
                  vx.ld % V == 0 && vy.ld % V == 0,
              0, 1.0, 1, epsilon};
    return dispatch(x->dtype, RowOp::LayerNorm, a);
}

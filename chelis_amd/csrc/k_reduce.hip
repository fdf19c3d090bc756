// Reductions over one axis on gfx950: sum (canonical tree), max, min
// ([05-OP-12/13]), argmax, argmin ([05-OP-15/16]), sum and max with an
// optional inlined FusedElem chain as the leaf (the reference's
// reduce_fused), prod (the C lane's left fold), plus the Bool8 count
// ([05-OP-29]).
//
// The reduced tensor is viewed as [outer, n, inner]. The canonical tree
// over n leaves equals a full binary tree over the leaves padded to a power
// of two with the operation's exact identity (-0 for +, -inf/+inf for
// max/min, never selected), so it can be evaluated hierarchically:
// each pass reduces aligned groups of G = 2^g consecutive leaves to one
// partial, and the next pass treats the partials as leaves, until one
// value per output remains. Every group is an aligned subtree, so the
// composition is the canonical tree bit for bit.
//
// Pass kernels:
//  * rows  (inner == 1): one wave per group of G = 64*S leaves; lane l
//    holds leaf s*64 + l of each segment s (coalesced loads), the wave64
//    butterfly builds each segment's 64-leaf subtree, then a tree over the
//    S segments.
//  * rows, contiguous (every input's leaves at stride 1, rows 16-byte
//    aligned): one wave per group of G = 64*V*S leaves, V = 16/sizeof(T);
//    lane l holds the V consecutive leaves 64V*s + V*l .. of segment s,
//    read with one 16-byte load per input. The in-lane tree over them is an
//    aligned V-leaf subtree; the butterfly joins 64 of those.
//  * cols  (inner > 1): one thread per (group, column), adjacent threads on
//    adjacent columns (coalesced); the thread loads its G = 32 leaves and
//    reduces them with an unrolled in-register tree.
// max/min/argmax combine in index order (lower lane / earlier leaf on the
// left), so first-NaN and first-index tie rules hold.
#include <algorithm>
#include <mutex>

#include "chain.h"

namespace chelis {
namespace {

// Every kernel in this file runs 256 threads per workgroup; grid-stride
// index arithmetic uses the constant, not blockDim.x (a vector load from
// the dispatch packet at the start of each wave).
constexpr int kReduceThreads = 256;

enum class Rk : int { Sum, Max, Min, ArgMax, ArgMin };

template <typename T, Rk K>
__device__ inline T identity() {
    if constexpr (K == Rk::Sum) return T(-0.0);
    if constexpr (K == Rk::Max || K == Rk::ArgMax) return -__builtin_huge_val();
    return __builtin_huge_val();
}

// combine(left, right) with left covering the earlier leaves.
template <typename T, Rk K>
__device__ inline void combine(T &a, int64_t &ia, T b, int64_t ib) {
    if constexpr (K == Rk::Sum) {
        a = a + b;
    } else {
        if (a != a) return;
        if (b != b) {
            a = b;
            ia = ib;
            return;
        }
        const bool take = (K == Rk::Max || K == Rk::ArgMax) ? (b > a) : (b < a);
        if (take) {
            a = b;
            ia = ib;
        }
    }
}

constexpr bool has_index(Rk k) { return k == Rk::ArgMax || k == Rk::ArgMin; }

// Leaf source: either the chain over the inputs or one plain input.
struct LeafSrc {
    int32_t n_in;
    const void *p[CHELIS_FUSED_MAX_INPUTS];
    int64_t so[CHELIS_FUSED_MAX_INPUTS], sn[CHELIS_FUSED_MAX_INPUTS], si[CHELIS_FUSED_MAX_INPUTS];
    const int64_t *idx;  // partial indices of a previous pass (argmax/argmin), or null
    int32_t join;        // rows: groups per row (2 or 4) joined inside the workgroup, or 0
};

// A chain leaf runs on the element's row of LDS slots (run_chain).
template <typename T, bool CHAIN>
__device__ inline T leaf(const ChainDev &ch, const LeafSrc &src, T *slot, int64_t o, int64_t i, int64_t j) {
    if constexpr (!CHAIN) {
        // nontemporal: each leaf is read once ([16384,4096] column sum 54 -> 49 us)
        return __builtin_nontemporal_load(static_cast<const T *>(src.p[0]) + (o * src.so[0] + i * src.sn[0] + j * src.si[0]));
    } else {
        T in[CHELIS_FUSED_MAX_INPUTS];
#pragma unroll
        for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k)
            if (k < src.n_in) in[k] = static_cast<const T *>(src.p[k])[o * src.so[k] + i * src.sn[k] + j * src.si[k]];
#pragma unroll
        for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k)
            if (k < src.n_in) slot[k] = in[k];
        return run_chain<T>(ch, slot);
    }
}

// Wave64 butterfly over one value (and index) per lane: lane l ends with the
// combination of the 64 lanes' values in lane order (the lower lane is
// always the left operand, so first-NaN and first-index rules hold).
template <typename T, Rk K>
__device__ inline void wave_join(T &v, int64_t &vi, int lane) {
    if constexpr (K == Rk::Sum) {
        v = wave_tree_sum(v);
        return;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        T ov = shfl_xor(v, m);
        int64_t oi = has_index(K) ? shfl_xor(vi, m) : 0;
        if (lane & m) {
            T a = ov;
            int64_t ia = oi;
            combine<T, K>(a, ia, v, vi);
            v = a;
            vi = ia;
        } else {
            combine<T, K>(v, vi, ov, oi);
        }
    }
}

// Tree over n (a power of two) values with their indices, in order.
template <typename T, Rk K, int N>
__device__ inline void ordered_tree(T (&v)[N], int64_t (&vi)[N]) {
#pragma unroll
    for (int w = N; w > 1; w >>= 1)
#pragma unroll
        for (int t = 0; t < w / 2; ++t) {
            T a = v[2 * t];
            int64_t ia = vi[2 * t];
            combine<T, K>(a, ia, v[2 * t + 1], vi[2 * t + 1]);
            v[t] = a;
            vi[t] = ia;
        }
}

template <typename T, Rk K>
__device__ inline T finalize(T v) {
    if constexpr (K == Rk::Sum) return canon(v);
    return v;
}

// out layout of a pass: [outer, groups, inner] values (+ i64 indices).
template <typename T, Rk K, int S, bool CHAIN>
__global__ __launch_bounds__(256) void reduce_rows_kernel(ChainDev ch, LeafSrc src, int64_t outer, int64_t n,
                                                          int64_t groups, T *__restrict__ out_v,
                                                          int64_t *__restrict__ out_i, bool last) {
    constexpr int G = 64 * S;
    __shared__ T slots[CHAIN ? 256 * kSlotStride : 1];
    T *slot = slots + (CHAIN ? threadIdx.x * kSlotStride : 0);
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= outer * groups) return;
    const int64_t o = item / groups, g = item % groups;
    T seg[S];
    int64_t sidx[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int64_t i = g * G + (int64_t)s * 64 + lane;
        T v = identity<T, K>();
        int64_t vi = i;
        if (i < n) {
            v = leaf<T, CHAIN>(ch, src, slot, o, i, 0);
            if (has_index(K) && src.idx) vi = src.idx[o * n + i];
        }
        wave_join<T, K>(v, vi, lane);
        seg[s] = v;
        sidx[s] = vi;
    }
    ordered_tree<T, K, S>(seg, sidx);
    if (lane == 0) {
        out_v[item] = last ? finalize<T, K>(seg[0]) : seg[0];
        if (has_index(K)) out_i[item] = sidx[0];
    }
}

// Contiguous rows: leaf i of row o of input k at p[k] + o*so[k] + i, each
// row start 16-byte aligned. Leaf indices are positions (a first pass, or a
// later pass of a value-only reduction). A chain leaf with NIN > 0 inputs
// (the count fixed at compile time) issues the 16-byte loads of all S
// segments before the first segment's interpreter run, so a wave holds
// S * NIN * 1 KiB in flight; NIN = 0 takes the input count at run time with
// one segment per wave.
template <typename T, Rk K, int S, bool CHAIN, int NIN = 0>
__global__ __launch_bounds__(256) void reduce_rows_vec_kernel(ChainDev ch, LeafSrc src, int64_t outer, int64_t n,
                                                              int64_t groups, T *__restrict__ out_v,
                                                              int64_t *__restrict__ out_i, bool last) {
    constexpr int V = 16 / sizeof(T);
    constexpr int G = 64 * V * S;
    constexpr int NI = NIN > 0 ? NIN : CHELIS_FUSED_MAX_INPUTS;
    static_assert(!CHAIN || NIN > 0 || S == 1, "a run-time input count takes one segment per wave");
    using Q = typename Vec16F<T>::type;
    // a chain leaf runs on the vector interpreter (run_chain_vec): its
    // slots are this launch's dynamic LDS, each thread's own
    extern __shared__ __align__(16) unsigned char red_lds[];
    Q *qs = reinterpret_cast<Q *>(red_lds);
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= outer * groups) return;
    const int64_t o = item / groups, g = item % groups;
    T v[CHAIN ? 1 : S][V];
    Q in[CHAIN ? S : 1][CHAIN ? NI : 1];
    if constexpr (CHAIN) {
        // every segment's loads issued before the first interpreter run
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int64_t i0 = g * G + (int64_t)s * 64 * V + (int64_t)lane * V;
#pragma unroll
            for (int k = 0; k < NI; ++k) {
                if (NIN > 0 || k < src.n_in) {
                    const T *p = static_cast<const T *>(src.p[k]) + o * src.so[k];
                    if (i0 + V <= n) {
                        in[s][k] = load_nt16(p + i0);
                    } else {
#pragma unroll
                        for (int e = 0; e < V; ++e)
                            reinterpret_cast<T *>(&in[s][k])[e] = i0 + e < n ? p[i0 + e] : T(0);
                    }
                }
            }
        }
    }
    if constexpr (!CHAIN) {
        // every load issued before the first combine
        const T *row = static_cast<const T *>(src.p[0]) + o * src.so[0];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int64_t i0 = g * G + (int64_t)s * 64 * V + (int64_t)lane * V;
            if (i0 + V <= n) {
                const Q q = load_nt16(row + i0);
                const T *qe = reinterpret_cast<const T *>(&q);
#pragma unroll
                for (int e = 0; e < V; ++e) v[s][e] = qe[e];
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) v[s][e] = i0 + e < n ? row[i0 + e] : identity<T, K>();
            }
        }
    }
    if constexpr (!CHAIN && (K == Rk::Max || K == Rk::Min)) {
        // Plain v_max (of the negated leaves for min) gives the [05-OP-12]
        // bits whenever the group holds no NaN and its extremum is not a
        // zero: a nonzero non-NaN value has one representation. Otherwise
        // the ordered combine below runs on the same registers.
        constexpr T sgn = K == Rk::Max ? T(1) : T(-1);
        T m = sgn * v[0][0];
        bool nan = false;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int e = 0; e < V; ++e) {
                m = vmax(m, sgn * v[s][e]);
                nan |= v[s][e] != v[s][e];
            }
        m = wave_vmax(m);
        if (!__any(nan) && m != T(0)) {
            if (lane == 0) out_v[item] = sgn * m;
            return;
        }
    }
    T seg[S];
    int64_t sidx[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int64_t i0 = g * G + (int64_t)s * 64 * V + (int64_t)lane * V;
        T(&cur)[V] = v[CHAIN ? 0 : s];
        if constexpr (CHAIN) {
#pragma unroll
            for (int k = 0; k < NI; ++k)
                if (NIN > 0 || k < src.n_in) qs[k * 256 + threadIdx.x] = in[s][k];
            T r[V];
            run_chain_vec<T, V>(ch, qs, NIN > 0 ? NIN : src.n_in, threadIdx.x, r);
#pragma unroll
            for (int e = 0; e < V; ++e) cur[e] = i0 + e < n ? r[e] : identity<T, K>();
        }
        int64_t vi[V];
#pragma unroll
        for (int e = 0; e < V; ++e) vi[e] = i0 + e;
        ordered_tree<T, K, V>(cur, vi);
        T x = cur[0];
        int64_t xi = vi[0];
        wave_join<T, K>(x, xi, lane);
        seg[s] = x;
        sidx[s] = xi;
    }
    ordered_tree<T, K, S>(seg, sidx);
    if constexpr (CHAIN && NIN > 0 && !has_index(K)) {
        if (src.join) {
            // The row's join groups are this workgroup's consecutive waves
            // (every item in range): their totals are the leaves of the
            // row's top subtree, joined in order and stored as the result.
            __shared__ T jv[4];
            if (lane == 0) jv[threadIdx.x >> 6] = seg[0];
            __syncthreads();
            const int w = threadIdx.x >> 6;
            if (lane == 0 && w % src.join == 0) {
                T a[4] = {jv[w], jv[w + 1], identity<T, K>(), identity<T, K>()};
                int64_t ia[4] = {0, 0, 0, 0};
                if (src.join == 4) {
                    a[2] = jv[2];
                    a[3] = jv[3];
                    ordered_tree<T, K, 4>(a, ia);
                } else {
                    combine<T, K>(a[0], ia[0], a[1], ia[1]);
                }
                out_v[item / src.join] = finalize<T, K>(a[0]);
            }
            return;
        }
    }
    if (lane == 0) {
        out_v[item] = last ? finalize<T, K>(seg[0]) : seg[0];
        if (has_index(K)) out_i[item] = sidx[0];
    }
}

template <typename T, Rk K, bool CHAIN>
__global__ __launch_bounds__(256) void reduce_cols_kernel(ChainDev ch, LeafSrc src, int64_t outer, int64_t n,
                                                          int64_t inner, int64_t groups, T *__restrict__ out_v,
                                                          int64_t *__restrict__ out_i, bool last) {
    constexpr int G = 32;
    __shared__ T slots[CHAIN ? 256 * kSlotStride : 1];
    T *slot = slots + (CHAIN ? threadIdx.x * kSlotStride : 0);
    const int64_t total = outer * groups * inner;
    const int64_t stride = (int64_t)gridDim.x * kReduceThreads;
    for (int64_t t = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x; t < total; t += stride) {
        const int64_t j = t % inner;
        const int64_t og = t / inner;
        const int64_t g = og % groups, o = og / groups;
        T v[G];
        int64_t vi[G];
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const int64_t i = g * G + q;
            v[q] = identity<T, K>();
            vi[q] = i;
            if (i < n) {
                v[q] = leaf<T, CHAIN>(ch, src, slot, o, i, j);
                if (has_index(K) && src.idx) vi[q] = src.idx[(o * n + i) * inner + j];
            }
        }
        ordered_tree<T, K, G>(v, vi);
        out_v[t] = last ? finalize<T, K>(v[0]) : v[0];
        if (has_index(K)) out_i[t] = vi[0];
    }
}

// Columns with inner >= 64, four waves per block on the same 64 columns:
// wave w reduces leaf group 4*gb + w (32 leaves, as reduce_cols_kernel
// does) and the four group totals join in LDS in order, so one block writes
// the total of an aligned 128-leaf group: fewer passes and partials.
template <typename T, Rk K, bool CHAIN>
__global__ __launch_bounds__(256) void reduce_cols4_kernel(ChainDev ch, LeafSrc src, int64_t outer, int64_t n,
                                                           int64_t inner, int64_t groups, T *__restrict__ out_v,
                                                           int64_t *__restrict__ out_i, bool last) {
    constexpr int G = 32;
    __shared__ T pv[4][64];
    __shared__ int64_t pi[has_index(K) ? 4 : 1][64];
    __shared__ T slots[CHAIN ? 256 * kSlotStride : 1];
    T *slot = slots + (CHAIN ? threadIdx.x * kSlotStride : 0);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t jblocks = (inner + 63) / 64;
    int64_t b = blockIdx.x;
    const int64_t jb = b % jblocks;
    b /= jblocks;
    const int64_t gb = b % groups, o = b / groups;
    const int64_t j = jb * 64 + lane;
    const bool jok = j < inner;
    T v[G];
    int64_t vi[G];
#pragma unroll
    for (int q = 0; q < G; ++q) {
        const int64_t i = (gb * 4 + w) * G + q;
        v[q] = identity<T, K>();
        vi[q] = i;
        if (jok && i < n) {
            v[q] = leaf<T, CHAIN>(ch, src, slot, o, i, j);
            if (has_index(K) && src.idx) vi[q] = src.idx[(o * n + i) * inner + j];
        }
    }
    ordered_tree<T, K, G>(v, vi);
    pv[w][lane] = v[0];
    if constexpr (has_index(K)) pi[w][lane] = vi[0];
    __syncthreads();
    if (w == 0 && jok) {
        T a[4];
        int64_t ia[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a[k] = pv[k][lane];
            ia[k] = has_index(K) ? pi[k][lane] : 0;
        }
        ordered_tree<T, K, 4>(a, ia);
        const int64_t t = (o * groups + gb) * inner + j;
        out_v[t] = last ? finalize<T, K>(a[0]) : a[0];
        if (has_index(K)) out_i[t] = ia[0];
    }
}

template <typename T>
__global__ void fill_kernel(T *p, int64_t n, T v) {
    const int64_t i = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x;
    if (i < n) p[i] = v;
}

// ProdReduce as the C lane computes it (crates/chelis-backend-c/src/emit.rs:
// 2551-2561 -> emit_reduce_simple, 8817-8912): `acc = 1; acc *= x[k]` over
// the axis in index order, a left fold rounded at the dtype after every
// multiply, the stored value NaN-finalized. The fold is sequential by
// definition (products do not reassociate bit for bit), so a thread owns one
// output; adjacent threads take adjacent columns (inner > 1) or adjacent rows.
// The reference HIP lane's reduce_prod folds the same way at f32 and f64
// (crates/chelis-backend-hip/src/kernels.rs:1888-1925).
template <typename T>
__global__ __launch_bounds__(256) void prod_fold_kernel(const T *__restrict__ x, int64_t outer, int64_t n,
                                                        int64_t inner, int64_t so, int64_t sn, int64_t si,
                                                        T *__restrict__ out) {
    const int64_t total = outer * inner;
    const int64_t stride = (int64_t)gridDim.x * kReduceThreads;
    for (int64_t t = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x; t < total; t += stride) {
        const int64_t o = t / inner, j = t % inner;
        const T *p = x + o * so + j * si;
        T acc = T(1);
        int64_t k = 0;
        // four loads in flight ahead of the dependent multiplies
        for (; k + 4 <= n; k += 4) {
            const T a0 = p[k * sn], a1 = p[(k + 1) * sn], a2 = p[(k + 2) * sn], a3 = p[(k + 3) * sn];
            acc = acc * a0;
            acc = acc * a1;
            acc = acc * a2;
            acc = acc * a3;
        }
        for (; k < n; ++k) acc = acc * p[k * sn];
        out[t] = canon(acc);
    }
}

// count: Bool8 leaves, exact i64 sums (any order gives the same integer),
// a byte other than 0/1 raises the reference kernel's error code 1.
__global__ __launch_bounds__(256) void count_kernel(const uint8_t *__restrict__ x, int64_t outer, int64_t n,
                                                    int64_t inner, int64_t so, int64_t sn, int64_t si,
                                                    int64_t *__restrict__ out, int32_t *__restrict__ err) {
    const int64_t total = outer * inner;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= total) return;
    const int64_t o = t / inner, j = t % inner;
    int64_t c = 0;
    bool bad = false;
    for (int64_t i = lane; i < n; i += 64) {
        const uint8_t b = x[o * so + i * sn + j * si];
        bad |= b > 1;
        c += b & 1;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) c += shfl_xor(c, m);
    if (bad) atomicOr(err, 1);
    if (lane == 0) out[t] = c;
}

// count over contiguous rows (16-byte aligned starts): each lane reads 16
// bytes per access; a byte's low bit is its count and any higher bit marks
// a byte other than 0/1.
__global__ __launch_bounds__(256) void count_rows_vec_kernel(const uint8_t *__restrict__ x, int64_t rows,
                                                             int64_t n, int64_t so, int64_t *__restrict__ out,
                                                             int32_t *__restrict__ err) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= rows) return;
    const uint8_t *r = x + t * so;
    const int64_t nv = n / 16;
    int64_t c = 0;
    uint32_t bad = 0;
#pragma unroll 4
    for (int64_t v = lane; v < nv; v += 64) {
        typedef uint32_t U4 __attribute__((ext_vector_type(4)));
        const U4 w = __builtin_nontemporal_load(reinterpret_cast<const U4 *>(r) + v);  // read once
        bad |= (w.x | w.y | w.z | w.w) & 0xFEFEFEFEu;
        c += __popc(w.x & 0x01010101u) + __popc(w.y & 0x01010101u) + __popc(w.z & 0x01010101u) +
             __popc(w.w & 0x01010101u);
    }
    for (int64_t i = nv * 16 + lane; i < n; i += 64) {
        const uint8_t b = r[i];
        bad |= b & 0xFEu;
        c += b & 1;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) c += shfl_xor(c, m);
    if (bad) atomicOr(err, 1);
    if (lane == 0) out[t] = c;
}

// ---------------------------------------------------------------- host
// Collapse the axes before `axis` into one stride and after it into one.
bool split3(const chelis_gpu_tensor *t, int32_t axis, int64_t *so, int64_t *sn, int64_t *si) {
    auto fold = [&](int32_t lo, int32_t hi, int64_t *st) {
        int64_t expect = -1;
        *st = 0;
        for (int32_t a = hi - 1; a >= lo; --a) {
            if (t->shape[a] == 1) continue;
            if (expect < 0) {
                *st = t->strides[a];
                expect = t->strides[a] * t->shape[a];
            } else {
                if (t->strides[a] != expect) return false;
                expect *= t->shape[a];
            }
        }
        return true;
    };
    *sn = t->shape[axis] == 1 ? 0 : t->strides[axis];
    return fold(0, axis, so) && fold(axis + 1, t->rank, si);
}

// An inlined FusedElem leaf exists only for Sum and Max, the two
// reductions fuse.rs folds a chain into (crates/chelis-dag-core/src/fuse.rs:463-487).
template <Rk K>
constexpr bool kChainable = K == Rk::Sum || K == Rk::Max;

// One pass of a reduction, planned on the host before anything is enqueued.
struct Pass {
    bool vec;       // contiguous rows with 16-byte loads
    int S;          // rows: segments per wave
    bool cols4;     // columns: four waves per 128-leaf group
    int64_t n;      // leaves per output this pass
    int64_t groups; // partials per output it writes
    int join = 0;   // rows, chain leaves: 2 or 4 groups joined in the workgroup, the pass writing the result
};
constexpr int kMaxPasses = 16;
// Contiguous chain leaves: the input counts with a compile-time instance
// whose loads for up to kChainSegments segments per wave are all issued
// before the interpreter runs.
constexpr int kChainPreloadInputs = 3;
constexpr int kChainSegments = 4;

// The pass sequence: partials of pass i are the leaves of pass i + 1 and
// live in a buffer 256-byte aligned, so their row alignment depends only
// on the row length. Returns the number of passes.
template <typename T, Rk K>
int plan_passes(const ChainDev &ch, bool chain, const LeafSrc &src, int64_t outer, int64_t n, int64_t inner,
                Pass (&passes)[kMaxPasses]) {
    const bool rows = inner == 1;
    int64_t cur_n = n;
    for (int i = 0; i < kMaxPasses; ++i) {
        const bool first = i == 0;
        const bool use_chain = first && chain;
        // contiguous rows take 16-byte loads: leaves at stride 1, row
        // starts aligned, and leaf indices that are positions
        bool vec = rows && !(has_index(K) && !first);
        if (first) {
            for (int32_t k = 0; vec && k < src.n_in; ++k)
                vec = src.sn[k] == 1 && (reinterpret_cast<uintptr_t>(src.p[k]) & 15u) == 0 &&
                      (src.so[k] * (int64_t)sizeof(T)) % 16 == 0;
        } else {
            vec = vec && (cur_n * (int64_t)sizeof(T)) % 16 == 0;
        }
        const int n_in = first ? src.n_in : 1;
        const size_t chain_lds = (size_t)(n_in + ch.n_steps) * 256 * 16;
        if (use_chain && chain_lds > 65536) vec = false;
        const int64_t unit = vec ? 64 * (16 / (int64_t)sizeof(T)) : 64;
        // rows: a row that fits one wave's 16 segments finishes in this pass;
        // a longer one is cut into as many groups as keep >= 1024 waves busy
        // (S = 16 only when there are rows enough), since a pass over few long
        // groups runs on a handful of waves. A contiguous chain leaf over up
        // to kChainPreloadInputs inputs takes up to kChainSegments segments
        // per wave (the interpreter is inlined once per segment), over more
        // inputs one.
        const int smax = vec && use_chain ? (src.n_in <= kChainPreloadInputs ? kChainSegments : 1) : 16;
        int S = 1;
        if (rows) {
            if (cur_n <= unit * smax) {
                while (unit * S < cur_n) S <<= 1;
            } else {
                while (S < smax && outer * ((cur_n + 2 * unit * S - 1) / (2 * unit * S)) >= 1024) S <<= 1;
            }
        }
        // columns: 128-leaf groups per block when 64 columns fill a wave
        const bool cols4 = !rows && inner >= 64 && grid_fits(outer * ((cur_n + 127) / 128) * ((inner + 63) / 64), 256);
        const int64_t G = rows ? unit * S : (cols4 ? 128 : 32);
        const int64_t groups = (cur_n + G - 1) / G;
        passes[i] = Pass{vec, S, cols4, cur_n, groups};
        if (groups == 1) return i + 1;
        // a contiguous chain leaf over 2 or 4 groups per row, rows filling
        // whole workgroups: the workgroup joins each row's groups itself
        // (no second launch)
        if (rows && vec && use_chain && !has_index(K) && S == kChainSegments && src.n_in <= kChainPreloadInputs &&
            (groups == 2 || groups == 4) && (outer * groups) % 4 == 0) {
            passes[i].join = (int)groups;
            return i + 1;
        }
        cur_n = groups;
    }
    return kMaxPasses;  // unreachable: each pass divides the leaves by >= 32
}

// Bytes of partials a plan needs: passes alternate between two value
// buffers (and two index buffers for argmax / argmin), each sized by the
// largest pass that writes it. Fills the four sizes when sizes != null.
template <typename T, Rk K>
size_t partial_bytes(const Pass *passes, int np, int64_t outer, int64_t inner, size_t *sizes = nullptr) {
    size_t need[4] = {0, 0, 0, 0};  // values A, values B, indices A, indices B
    for (int i = 0; i < np; ++i) {
        const bool last = i + 1 == np;
        const size_t cells = (size_t)(outer * passes[i].groups * inner);
        const int b = i & 1;
        // the last pass writes the result, except the values of argmax /
        // argmin, whose result is the index
        if (!last || has_index(K)) need[b] = std::max(need[b], ((cells * sizeof(T)) + 255) & ~size_t(255));
        if (has_index(K) && !last)
            need[2 + b] = std::max(need[2 + b], ((cells * sizeof(int64_t)) + 255) & ~size_t(255));
    }
    if (sizes)
        for (int k = 0; k < 4; ++k) sizes[k] = need[k];
    return need[0] + need[1] + need[2] + need[3];
}

// Where pass partials live: the library's stream-ordered cached scratch
// (region == null), or a caller-fixed device region carved in order.
struct PartialStore {
    char *region = nullptr;
    size_t region_bytes = 0;
};

// Cached-scratch blocks held for one reduction, returned in stream order.
struct HeldScratch {
    void *p[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t bytes[4] = {0, 0, 0, 0};
    ~HeldScratch() {
        for (int k = 0; k < 4; ++k) scratch_free(p[k], bytes[k]);
    }
};

template <typename T, Rk K>
int32_t run_reduce(const ChainDev &ch, bool chain, LeafSrc src, int64_t outer, int64_t n, int64_t inner,
                   void *out, hipStream_t st, const PartialStore &store) {
    if (chain && !kChainable<K>) return set_error(CHELIS_HIP_EUNSUPPORTED, "reduce: a fused leaf chain feeds sum or max only");
    Pass passes[kMaxPasses];
    const int np = plan_passes<T, K>(ch, chain, src, outer, n, inner, passes);
    size_t sizes[4];
    const size_t total = partial_bytes<T, K>(passes, np, outer, inner, sizes);
    void *buf[4] = {nullptr, nullptr, nullptr, nullptr};
    HeldScratch held;
    if (store.region) {
        if (total > store.region_bytes)
            return set_error(CHELIS_HIP_EDOMAIN, "reduce: the passes need %zu bytes of partials, the static scratch holds %zu",
                             total, store.region_bytes);
        size_t off = 0;
        for (int k = 0; k < 4; ++k) {
            buf[k] = sizes[k] ? store.region + off : nullptr;
            off += sizes[k];
        }
    } else {
        for (int k = 0; k < 4; ++k) {
            if (!sizes[k]) continue;
            held.bytes[k] = sizes[k];
            if (!(held.p[k] = buf[k] = scratch_alloc(sizes[k])))
                return set_error(CHELIS_HIP_EHIP, "reduce: scratch allocation failed");
        }
    }
    const bool rows = inner == 1;
    T *prev_v = nullptr;
    int64_t *prev_i = nullptr;
    for (int pi = 0; pi < np; ++pi) {
        const Pass &ps = passes[pi];
        const bool first = pi == 0;
        const int64_t cur_n = ps.n, groups = ps.groups;
        const bool vec = ps.vec, cols4 = ps.cols4;
        const int S = ps.S;
        LeafSrc s = src;
        s.join = ps.join;
        if (!first) {
            s.n_in = 1;
            s.p[0] = prev_v;
            s.so[0] = cur_n * inner;
            s.sn[0] = inner;
            s.si[0] = 1;
            s.idx = prev_i;
        }
        const bool use_chain = first && chain;
        const size_t chain_lds = (size_t)(s.n_in + ch.n_steps) * 256 * 16;
        const bool last = pi + 1 == np;
        const int64_t cells = outer * groups * inner;
        T *dst_v;
        int64_t *dst_i = nullptr;
        if (last) {
            dst_v = has_index(K) ? nullptr : static_cast<T *>(out);
            dst_i = has_index(K) ? static_cast<int64_t *>(out) : nullptr;
        } else {
            dst_v = static_cast<T *>(buf[pi & 1]);
            dst_i = static_cast<int64_t *>(buf[2 + (pi & 1)]);
        }
        // the index-only result of argmax / argmin still needs value partials
        if (!dst_v) dst_v = static_cast<T *>(buf[pi & 1]);
        if (rows) {
            const unsigned grid = grid_for(outer * groups, 4);
            if (!grid_fits(grid, 256)) return set_error(CHELIS_HIP_EUNSUPPORTED, "reduce: too many row groups");
#define CHELIS_ROWS_LAUNCH(KERNEL, SS, CHAIN_OK, LDS)                                                        \
    if constexpr (kChainable<K> && (CHAIN_OK)) {                                                              \
        if (use_chain) {                                                                                      \
            KERNEL<T, K, SS, true><<<grid, 256, LDS, st>>>(ch, s, outer, cur_n, groups, dst_v, dst_i, last);  \
            break;                                                                                            \
        }                                                                                                     \
    }                                                                                                         \
    KERNEL<T, K, SS, false><<<grid, 256, 0, st>>>(ch, s, outer, cur_n, groups, dst_v, dst_i, last);           \
    break;
#define CHELIS_ROWS_CASE(SS)                                                                                  \
    case SS:                                                                                                  \
        if (vec) {                                                                                            \
            if constexpr (kChainable<K> && SS > 1 && SS <= kChainSegments) {                                 \
                if (use_chain) {                                                                              \
                    if (s.n_in == 1)                                                                          \
                        reduce_rows_vec_kernel<T, K, SS, true, 1>                                             \
                            <<<grid, 256, chain_lds, st>>>(ch, s, outer, cur_n, groups, dst_v, dst_i, last);  \
                    else if (s.n_in == 2)                                                                     \
                        reduce_rows_vec_kernel<T, K, SS, true, 2>                                             \
                            <<<grid, 256, chain_lds, st>>>(ch, s, outer, cur_n, groups, dst_v, dst_i, last);  \
                    else if (s.n_in == 3)                                                                     \
                        reduce_rows_vec_kernel<T, K, SS, true, 3>                                             \
                            <<<grid, 256, chain_lds, st>>>(ch, s, outer, cur_n, groups, dst_v, dst_i, last);  \
                    else                                                                                      \
                        return set_error(CHELIS_HIP_EDOMAIN, "reduce: internal chain plan, %d inputs over %d segments", \
                                         s.n_in, SS);                                                         \
                    break;                                                                                    \
                }                                                                                             \
            }                                                                                                 \
            CHELIS_ROWS_LAUNCH(reduce_rows_vec_kernel, SS, SS == 1, chain_lds)                                \
        }                                                                                                     \
        CHELIS_ROWS_LAUNCH(reduce_rows_kernel, SS, true, 0)
            switch (S) {
                CHELIS_ROWS_CASE(1)
                CHELIS_ROWS_CASE(2)
                CHELIS_ROWS_CASE(4)
                CHELIS_ROWS_CASE(8)
                CHELIS_ROWS_CASE(16)
                default: return set_error(CHELIS_HIP_EDOMAIN, "reduce: internal segment count %d", S);
            }
#undef CHELIS_ROWS_CASE
#undef CHELIS_ROWS_LAUNCH
        } else if (cols4) {
            const unsigned grid = (unsigned)(outer * groups * ((inner + 63) / 64));
            bool done = false;
            if constexpr (kChainable<K>) {
                if (use_chain) {
                    reduce_cols4_kernel<T, K, true><<<grid, 256, 0, st>>>(ch, s, outer, cur_n, inner, groups, dst_v,
                                                                          dst_i, last);
                    done = true;
                }
            }
            if (!done)
                reduce_cols4_kernel<T, K, false><<<grid, 256, 0, st>>>(ch, s, outer, cur_n, inner, groups, dst_v, dst_i,
                                                                       last);
        } else {
            int64_t blocks = (cells + 255) / 256;
            if (blocks > 16384) blocks = 16384;
            bool done = false;
            if constexpr (kChainable<K>) {
                if (use_chain) {
                    reduce_cols_kernel<T, K, true><<<(unsigned)blocks, 256, 0, st>>>(ch, s, outer, cur_n, inner, groups,
                                                                                     dst_v, dst_i, last);
                    done = true;
                }
            }
            if (!done)
                reduce_cols_kernel<T, K, false><<<(unsigned)blocks, 256, 0, st>>>(ch, s, outer, cur_n, inner, groups,
                                                                                  dst_v, dst_i, last);
        }
        CHELIS_LAUNCH_CHECK();
        prev_v = dst_v;
        prev_i = dst_i;
    }
    return CHELIS_HIP_OK;
}

template <typename T>
int32_t dispatch_kind(int32_t op, const ChainDev &ch, bool chain, const LeafSrc &src, int64_t outer, int64_t n,
                      int64_t inner, void *out, hipStream_t st, const PartialStore &store) {
    switch (op) {
        case CHELIS_REDUCE_SUM: return run_reduce<T, Rk::Sum>(ch, chain, src, outer, n, inner, out, st, store);
        case CHELIS_REDUCE_MAX: return run_reduce<T, Rk::Max>(ch, chain, src, outer, n, inner, out, st, store);
        case CHELIS_REDUCE_MIN: return run_reduce<T, Rk::Min>(ch, chain, src, outer, n, inner, out, st, store);
        case CHELIS_REDUCE_ARGMAX: return run_reduce<T, Rk::ArgMax>(ch, chain, src, outer, n, inner, out, st, store);
        case CHELIS_REDUCE_ARGMIN: return run_reduce<T, Rk::ArgMin>(ch, chain, src, outer, n, inner, out, st, store);
        default: return set_error(CHELIS_HIP_EDOMAIN, "reduce: unknown op %d", op);
    }
}

int32_t load_chain(const chelis_fused_chain *chain, int32_t n_inputs, ChainDev *ch) {
    *ch = ChainDev{};
    if (!chain) return CHELIS_HIP_OK;
    if (chain->n_steps < 1 || chain->n_steps > CHELIS_FUSED_MAX_STEPS)
        return set_error(CHELIS_HIP_EDOMAIN, "chain: %d steps (1..%d)", chain->n_steps, CHELIS_FUSED_MAX_STEPS);
    ch->n_steps = chain->n_steps;
    for (int32_t i = 0; i < chain->n_steps; ++i) {
        const chelis_fused_step &st = chain->steps[i];
        if (st.op >= CHELIS_FUSED_COUNT_) return set_error(CHELIS_HIP_EDOMAIN, "chain: step %d op %d", i, st.op);
        for (int j = 0; j < 2; ++j) {
            const int32_t a = st.args[j];
            if ((a >= 0 && a >= n_inputs) || (a < 0 && -a - 1 >= i))
                return set_error(CHELIS_HIP_EDOMAIN, "chain: step %d arg %d out of range", i, j);
        }
        ch->op[i] = st.op;
        ch->a0[i] = (int8_t)st.args[0];
        ch->a1[i] = (int8_t)st.args[1];
        ch->imm[i] = st.imm;
    }
    return CHELIS_HIP_OK;
}

}  // namespace
}  // namespace chelis

using namespace chelis;

namespace chelis {
namespace {

int32_t reduce_entry(int32_t op, const chelis_fused_chain *chain, const chelis_gpu_tensor *const *inputs,
                     int32_t n_inputs, int32_t axis, const chelis_gpu_tensor *out, const PartialStore &store) {
    int32_t s;
    if (op == CHELIS_REDUCE_COUNT) return set_error(CHELIS_HIP_EDOMAIN, "reduce: use chelis_hip_count for counts");
    if (n_inputs < 1 || n_inputs > CHELIS_FUSED_MAX_INPUTS || !inputs)
        return set_error(CHELIS_HIP_EDOMAIN, "reduce: %d inputs", n_inputs);
    if (!chain && n_inputs != 1) return set_error(CHELIS_HIP_EDOMAIN, "reduce: a plain reduction takes one input");
    if ((s = check_tensor(out, "out"))) return s;
    const chelis_gpu_tensor *x0 = inputs[0];
    for (int32_t k = 0; k < n_inputs; ++k) {
        if ((s = check_tensor(inputs[k], "input"))) return s;
        if (!is_float(inputs[k]->dtype) || inputs[k]->dtype != x0->dtype || !same_shape(inputs[k], x0))
            return set_error(CHELIS_HIP_EDOMAIN, "reduce: inputs must share one f32/f64 dtype and shape");
    }
    const int32_t rank = x0->rank;
    if (axis < 0) axis += rank;
    if (axis < 0 || axis >= rank) return set_error(CHELIS_HIP_EDOMAIN, "reduce: axis out of range");
    const bool idx_out = op == CHELIS_REDUCE_ARGMAX || op == CHELIS_REDUCE_ARGMIN;
    if (out->dtype != (idx_out ? CHELIS_DTYPE_I64 : x0->dtype))
        return set_error(CHELIS_HIP_EDOMAIN, "reduce: result dtype must be %s", idx_out ? "i64" : "the input's");
    if (out->rank != rank - 1 || !is_contiguous(out))
        return set_error(CHELIS_HIP_EDOMAIN, "reduce: result must be contiguous with the axis removed");
    for (int32_t a = 0, b = 0; a < rank; ++a) {
        if (a == axis) continue;
        if (out->shape[b++] != x0->shape[a]) return set_error(CHELIS_HIP_EDOMAIN, "reduce: result shape mismatch");
    }
    ChainDev ch;
    if ((s = load_chain(chain, n_inputs, &ch))) return s;
    int64_t outer = 1, inner = 1;
    const int64_t n = x0->shape[axis];
    for (int32_t a = 0; a < axis; ++a) outer *= x0->shape[a];
    for (int32_t a = axis + 1; a < rank; ++a) inner *= x0->shape[a];
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    if (outer * inner == 0) return CHELIS_HIP_OK;
    if (n == 0) {
        if (op != CHELIS_REDUCE_SUM && op != CHELIS_REDUCE_PROD)
            return set_error(CHELIS_HIP_EDOMAIN, "numeric trap: domain in %s at %s",
                             op == CHELIS_REDUCE_MAX ? "max_reduce" : op == CHELIS_REDUCE_MIN ? "min_reduce"
                             : op == CHELIS_REDUCE_ARGMAX ? "argmax_reduce" : "argmin_reduce",
                             idx_out ? "i64" : (x0->dtype == CHELIS_DTYPE_F32 ? "f32" : "f64"));
        const unsigned grid = grid_for(out->count, 256);
        if (!grid_fits(grid, 256)) return set_error(CHELIS_HIP_EUNSUPPORTED, "reduce: too many results");
        if (x0->dtype == CHELIS_DTYPE_F32)
            fill_kernel<float><<<grid, 256, 0, st>>>((float *)out->data, out->count, op == CHELIS_REDUCE_SUM ? 0.0f : 1.0f);
        else
            fill_kernel<double><<<grid, 256, 0, st>>>((double *)out->data, out->count, op == CHELIS_REDUCE_SUM ? 0.0 : 1.0);
        CHELIS_LAUNCH_CHECK();
        return CHELIS_HIP_OK;
    }
    LeafSrc src{};
    src.n_in = n_inputs;
    for (int32_t k = 0; k < n_inputs; ++k) {
        src.p[k] = inputs[k]->data;
        if (!split3(inputs[k], axis, &src.so[k], &src.sn[k], &src.si[k]))
            return set_error(CHELIS_HIP_EUNSUPPORTED, "reduce: input %d axes do not collapse to [outer, n, inner]", k);
    }
    if (op == CHELIS_REDUCE_PROD) {
        if (chain) return set_error(CHELIS_HIP_EUNSUPPORTED, "reduce: a fused leaf chain feeds sum or max only");
        int64_t blocks = (outer * inner + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        if (x0->dtype == CHELIS_DTYPE_F32)
            prod_fold_kernel<float><<<(unsigned)blocks, 256, 0, st>>>((const float *)src.p[0], outer, n, inner,
                                                                       src.so[0], src.sn[0], src.si[0],
                                                                       (float *)out->data);
        else
            prod_fold_kernel<double><<<(unsigned)blocks, 256, 0, st>>>((const double *)src.p[0], outer, n, inner,
                                                                        src.so[0], src.sn[0], src.si[0],
                                                                        (double *)out->data);
        CHELIS_LAUNCH_CHECK();
        return CHELIS_HIP_OK;
    }
    return x0->dtype == CHELIS_DTYPE_F32
               ? dispatch_kind<float>(op, ch, chain != nullptr, src, outer, n, inner, out->data, st, store)
               : dispatch_kind<double>(op, ch, chain != nullptr, src, outer, n, inner, out->data, st, store);
}

}  // namespace
}  // namespace chelis

// The allocation-free reduce entry's pass partials: one fixed array per
// device, reached through its device address (the host-side name is only a
// stand-in). The address is looked up once per device, with that device
// current, and kept.
static __device__ __align__(256) unsigned char scratch[CHELIS_HIP_STATIC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_addr_mutex;
constexpr int kMaxScratchDevices = 64;
void *g_scratch_addr[kMaxScratchDevices] = {};

int32_t static_scratch_address(void **addr) {
    int device = -1;
    CHELIS_HIP_TRY(hipGetDevice(&device));
    if (device < 0 || device >= kMaxScratchDevices)
        return set_error(CHELIS_HIP_EHIP, "static scratch: device %d outside 0..%d", device, kMaxScratchDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_addr_mutex);
    if (!g_scratch_addr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(CHELIS_HIP_EHIP, "static scratch: hipGetSymbolAddress: %s", hipGetErrorString(e));
        g_scratch_addr[device] = p;
    }
    *addr = g_scratch_addr[device];
    return CHELIS_HIP_OK;
}
}  // namespace

extern "C" int32_t chelis_hip_reduce(int32_t op, const chelis_fused_chain *chain,
                                     const chelis_gpu_tensor *const *inputs, int32_t n_inputs, int32_t axis,
                                     const chelis_gpu_tensor *out) {
    return reduce_entry(op, chain, inputs, n_inputs, axis, out, PartialStore{});
}

extern "C" int32_t chelis_hip_reduce_static(int32_t op, const chelis_fused_chain *chain,
                                            const chelis_gpu_tensor *const *inputs, int32_t n_inputs, int32_t axis,
                                            const chelis_gpu_tensor *out) {
    void *addr = nullptr;
    if (int32_t s = static_scratch_address(&addr)) return s;
    PartialStore store;
    store.region = static_cast<char *>(addr);
    store.region_bytes = CHELIS_HIP_STATIC_SCRATCH_BYTES;
    return reduce_entry(op, chain, inputs, n_inputs, axis, out, store);
}

extern "C" int32_t chelis_hip_count(const chelis_gpu_tensor *x, int32_t axis, const chelis_gpu_tensor *out,
                                    int32_t *error_code) {
    int32_t s;
    if ((s = check_tensor(x, "x")) || (s = check_tensor(out, "out"))) return s;
    if (x->dtype != CHELIS_DTYPE_BOOL || out->dtype != CHELIS_DTYPE_I64)
        return set_error(CHELIS_HIP_EDOMAIN, "count: bool input and i64 result required");
    if (axis < 0) axis += x->rank;
    if (axis < 0 || axis >= x->rank) return set_error(CHELIS_HIP_EDOMAIN, "count: axis out of range");
    if (out->rank != x->rank - 1 || !is_contiguous(out))
        return set_error(CHELIS_HIP_EDOMAIN, "count: result must be contiguous with the axis removed");
    for (int32_t a = 0, b = 0; a < x->rank; ++a) {
        if (a == axis) continue;
        if (out->shape[b++] != x->shape[a]) return set_error(CHELIS_HIP_EDOMAIN, "count: result shape mismatch");
    }
    int64_t so, sn, si;
    if (!split3(x, axis, &so, &sn, &si))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "count: axes do not collapse to [outer, n, inner]");
    int64_t outer = 1, inner = 1;
    for (int32_t a = 0; a < axis; ++a) outer *= x->shape[a];
    for (int32_t a = axis + 1; a < x->rank; ++a) inner *= x->shape[a];
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    if (error_code) *error_code = 0;
    if (outer * inner == 0) return CHELIS_HIP_OK;
    int32_t *host = nullptr;
    int32_t *words = status_words(&host);
    if (!words) return set_error(CHELIS_HIP_EHIP, "count: no status word on this device");
    // with error_code: this call's own word, read back before returning;
    // without: the trap channel, read at the caller's entry end
    int32_t *err = error_code ? words : words + 1;
    if (error_code) CHELIS_HIP_TRY(hipMemsetAsync(err, 0, sizeof(int32_t), st));
    if (!grid_fits(grid_for(outer * inner, 4), 256)) return set_error(CHELIS_HIP_EUNSUPPORTED, "count: too many results");
    if (inner == 1 && sn == 1 && so % 16 == 0 && (reinterpret_cast<uintptr_t>(x->data) & 15u) == 0)
        count_rows_vec_kernel<<<grid_for(outer, 4), 256, 0, st>>>((const uint8_t *)x->data, outer, x->shape[axis], so,
                                                                  (int64_t *)out->data, err);
    else
        count_kernel<<<grid_for(outer * inner, 4), 256, 0, st>>>((const uint8_t *)x->data, outer, x->shape[axis],
                                                                 inner, so, sn, si, (int64_t *)out->data, err);
    CHELIS_LAUNCH_CHECK();
    if (!error_code) return CHELIS_HIP_OK;
    CHELIS_HIP_TRY(hipMemcpyAsync(host, err, sizeof(int32_t), hipMemcpyDeviceToHost, st));
    CHELIS_HIP_TRY(hipStreamSynchronize(st));
    *error_code = *host;
    return CHELIS_HIP_OK;
}

extern "C" int32_t chelis_hip_trap_status(int32_t *code) {
    hipStream_t st = chelis::stream();
    if (!st) return chelis::set_error(CHELIS_HIP_EHIP, "no HIP device");
    int32_t *host = nullptr;
    int32_t *words = chelis::status_words(&host);
    if (!words) return chelis::set_error(CHELIS_HIP_EHIP, "trap status: no status word on this device");
    CHELIS_HIP_TRY(hipMemcpyAsync(host, words + 1, sizeof(int32_t), hipMemcpyDeviceToHost, st));
    CHELIS_HIP_TRY(hipStreamSynchronize(st));
    const int32_t v = *host;
    if (v) {
        CHELIS_HIP_TRY(hipMemsetAsync(words + 1, 0, sizeof(int32_t), st));
        CHELIS_HIP_TRY(hipStreamSynchronize(st));
    }
    if (code) *code = v;
    return CHELIS_HIP_OK;
}

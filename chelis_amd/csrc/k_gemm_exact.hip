// Canonical-tree matmul kernels: every output is the [05-OP-30]
// adjacent-pair tree over its K products, as the reference C lane computes
// it (crates/chelis-backend-c/src/emit.rs:8431-8560, the inlined product),
// so these results are bit-exact with the C backend. They serve the shapes
// the north star routes away from the matrix cores (GEMV, narrow outputs,
// short K) and every shape under CHELIS_MATMUL_EXACT.
//
// Tree decomposition. The canonical tree over K leaves equals the full
// binary tree over the leaves padded with -0.0 (the exact additive
// identity) to any power of two >= K; a full tree over aligned blocks of
// 2^b leaves is the full tree over the block totals; and the streamed carry
// tree over the block totals (a completed subtree of 2^d blocks waits in
// level d; block c first absorbs one waiting subtree per trailing one bit of
// c, the waiting one on the left; at the end the waiting subtrees fold
// lowest level first) is the canonical tree over those totals. So a kernel
// may cut K into aligned segments, reduce each segment as a full tree in any
// evaluation order that respects its pairing, and stream the segment totals
// through a carry stack.
//
// Inside a segment of 64*V leaves, lane l of a wave holds the V consecutive
// leaves l*V .. l*V+V-1: an in-register tree over V, then a wave64 butterfly
// (xor 1, 2, ..., 32) joins aligned lane blocks in increasing size. IEEE
// addition is commutative bit for bit, so the operand order of each join is
// free; the final NaN is canonicalized.
#include "gemm.h"

#include <algorithm>

namespace chelis {
namespace {

constexpr int MAXD = 24;  // carry-stack depth: up to 2^23 segments

// Push one block total into a wave-uniform carry stack of depth DEPTH (count
// = index of this block, below 2^DEPTH). Unrolled with static indices so
// the stack stays in VGPRs.
template <typename T, int DEPTH>
__device__ inline void carry_push(T (&lvl)[DEPTH], int64_t count, T carry) {
    bool done = false;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        if (!done) {
            if ((count >> d) & 1) {
                carry = lvl[d] + carry;
            } else {
                lvl[d] = carry;
                done = true;
            }
        }
    }
}

template <typename T, int DEPTH>
__device__ inline T carry_total(const T (&lvl)[DEPTH], int64_t count) {
    T total = T(0);
    bool found = false;
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        if ((count >> d) & 1) {
            total = found ? lvl[d] + total : lvl[d];
            found = true;
        }
    }
    return total;
}

template <typename T, int V>
__device__ inline T tree_v(T (&x)[V]) {
#pragma unroll
    for (int w = V; w > 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w / 2; ++i) x[i] = x[2 * i] + x[2 * i + 1];
    return x[0];
}

template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
    using type = float4;
    static constexpr int W = 4;
};
template <>
struct Vec16<double> {
    using type = double2;
    static constexpr int W = 2;
};

// V elements at p[0], p[s], ..., zero where k >= K; vector loads when the
// run is contiguous, aligned and complete (NT: streaming, read-once data).
template <typename T, int V, bool CONTIG, bool NT = false>
__device__ inline void load_run(const T *__restrict__ p, int64_t s, int64_t k, int64_t K, bool vec_ok, T (&x)[V]) {
    if (CONTIG && vec_ok && k + V <= K) {
        constexpr int W = Vec16<T>::W;
        typedef T nv __attribute__((ext_vector_type(Vec16<T>::W)));
#pragma unroll
        for (int q = 0; q < V / W; ++q) {
            nv v;
            if constexpr (NT) v = __builtin_nontemporal_load(reinterpret_cast<const nv *>(p) + q);
            else v = reinterpret_cast<const nv *>(p)[q];
#pragma unroll
            for (int u = 0; u < W; ++u) x[q * W + u] = v[u];
        }
    } else {
#pragma unroll
        for (int u = 0; u < V; ++u) x[u] = (k + u < K) ? p[CONTIG ? u : u * s] : T(0);
    }
}

// ---------------------------------------------------------------- wave per output
// GEMV-class shapes: one wave streams one output's K products, 64*V leaves
// per segment, fully coalesced when the operand is K-contiguous.
template <typename T, int V, bool AK, bool BK, int DEPTH>
__global__ __launch_bounds__(256) void tree_wave_kernel(GemmProblem p, int64_t outputs, bool a_vec, bool b_vec) {
    const int lane = threadIdx.x & 63;
    const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= outputs) return;  // whole waves leave together
    const int64_t n = w % p.N, mz = w / p.N, m = mz % p.M, z = mz / p.M;
    const int64_t z0 = z / p.nb1, z1 = z % p.nb1;
    const T *A = static_cast<const T *>(p.a) + z0 * p.sa0 + z1 * p.sa1 + m * p.sam;
    const T *B = static_cast<const T *>(p.b) + z0 * p.sb0 + z1 * p.sb1 + n * p.sbn;
    constexpr int SEG = 64 * V;
    const int64_t nseg = (p.K + SEG - 1) / SEG;
    T lvl[DEPTH];
    int64_t s = 0;
    if (AK && BK && a_vec && b_vec) {
        // whole segments of contiguous, aligned runs: branch-free vector
        // loads, the next segment's loads in flight while this one is summed
        // (the last prefetch is clamped to the last whole segment)
        // Layout: vector q of lane l holds the W leaves at 64W q + W l, so
        // each load instruction of the wave reads one contiguous 1 KiB run
        // (nontemporal: the matrix is read once). Quarter q of the segment,
        // [64W q, 64W (q + 1)), is an aligned subtree: W-leaf trees in the
        // lanes, joined across the wave, then the quarters in order.
        constexpr int W = Vec16<T>::W, NQ = V / W;
        typedef T nv __attribute__((ext_vector_type(W)));
        const int64_t nfull = p.K / SEG;
        T a0[V], b0[V], a1[V], b1[V];
        auto fetch = [&](int64_t seg, T(&a)[V], T(&b)[V]) {
            const int64_t k = (seg < nfull ? seg : nfull - 1) * SEG + (int64_t)lane * W;
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const nv va = __builtin_nontemporal_load(reinterpret_cast<const nv *>(A + k + q * 64 * W));
                const nv vb = *reinterpret_cast<const nv *>(B + k + q * 64 * W);
#pragma unroll
                for (int u = 0; u < W; ++u) a[q * W + u] = va[u], b[q * W + u] = vb[u];
            }
        };
        auto sum = [&](int64_t seg, T(&a)[V], const T(&b)[V]) {
            T quarter[NQ];
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                T x[W];
#pragma unroll
                for (int u = 0; u < W; ++u) x[u] = a[q * W + u] * b[q * W + u];
                quarter[q] = wave_tree_sum(tree_v<T, W>(x));
            }
            carry_push<T, DEPTH>(lvl, seg, tree_v<T, NQ>(quarter));
        };
        // unrolled by two so the two register sets swap roles without copies
        // (a copy of a prefetched set would wait for its loads at once)
        // (the scheduling barriers keep each prefetch ahead of the sum that
        // follows it: sunk below, its loads would be waited for at once)
        if (nfull > 0) fetch(0, a0, b0);
        for (; s + 1 < nfull; s += 2) {
            fetch(s + 1, a1, b1);
            __builtin_amdgcn_sched_barrier(0);
            sum(s, a0, b0);
            fetch(s + 2, a0, b0);
            __builtin_amdgcn_sched_barrier(0);
            sum(s + 1, a1, b1);
        }
        if (s < nfull) {
            sum(s, a0, b0);
            ++s;
        }
    }
    for (; s < nseg; ++s) {
        const int64_t k = s * SEG + (int64_t)lane * V;
        T a[V], b[V];
        load_run<T, V, AK>(A + k * p.sak, p.sak, k, p.K, a_vec, a);
        load_run<T, V, BK>(B + k * p.sbk, p.sbk, k, p.K, b_vec, b);
#pragma unroll
        for (int u = 0; u < V; ++u) a[u] = (k + u < p.K) ? a[u] * b[u] : T(-0.0);
        carry_push<T, DEPTH>(lvl, s, wave_tree_sum(tree_v<T, V>(a)));
    }
    if (lane == 0) {
        T *C = static_cast<T *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
        C[m * p.scm + n * p.scn] = gemm_epilogue<T>(carry_total<T, DEPTH>(lvl, nseg), p, z0, z1, m, n);
    }
}

// ---------------------------------------------------------------- tiled, narrow N
// A workgroup of WAVES waves owns WAVES*R rows x NJ columns. Per segment of
// 64*V leaves the NJ-column B panel is staged once in LDS (K-contiguous per
// column) and shared by every wave; each wave forms the in-lane trees of
// its P = R*NJ outputs and then runs a reduce-scatter butterfly: at step
// xor m a lane keeps the half of its outputs whose bit matches its own lane
// bit and receives the partner's partial of that half, so one shuffle per
// output pair replaces a full butterfly per output. After log2(P) steps
// lane l holds output l mod P; the remaining steps (xor P .. 32) are plain
// butterflies. The joins stay aligned lane blocks of increasing size, so the
// tree is unchanged. Each lane then streams its one output's segment totals
// through its own carry stack.
template <typename T, int V, int R, int NJ, int WAVES, bool AK, bool BKFAST>
__global__ __launch_bounds__(64 * WAVES) void tree_tiled_kernel(GemmProblem p, bool a_vec) {
    constexpr int P = R * NJ;
    static_assert((P & (P - 1)) == 0 && P <= 64, "outputs per wave must be a power of two <= 64");
    constexpr int SEG = 64 * V;
    constexpr int PAD = 16 / sizeof(T);
    constexpr int LDB = SEG + PAD;
    __shared__ __attribute__((aligned(16))) T Bs[NJ * LDB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t z = blockIdx.z;
    const int64_t z0 = z / p.nb1, z1 = z % p.nb1;
    const int64_t m_base = (int64_t)blockIdx.x * (WAVES * R) + wave * R;
    const int64_t n0 = (int64_t)blockIdx.y * NJ;
    const T *A = static_cast<const T *>(p.a) + z0 * p.sa0 + z1 * p.sa1;
    const T *B = static_cast<const T *>(p.b) + z0 * p.sb0 + z1 * p.sb1;
    const int64_t nseg = (p.K + SEG - 1) / SEG;
    T lvl[MAXD];
    for (int64_t s = 0; s < nseg; ++s) {
        const int64_t kseg = s * SEG;
        __syncthreads();
        for (int idx = threadIdx.x; idx < NJ * SEG; idx += 64 * WAVES) {
            const int kk = BKFAST ? idx % SEG : idx / NJ;
            const int j = BKFAST ? idx / SEG : idx % NJ;
            const int64_t gk = kseg + kk, gn = n0 + j;
            Bs[j * LDB + kk] = (gk < p.K && gn < p.N) ? B[gk * p.sbk + gn * p.sbn] : T(0);
        }
        __syncthreads();
        const int64_t k = kseg + (int64_t)lane * V;
        T a[R][V];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t m = m_base + r;
            if (m < p.M) {
                load_run<T, V, AK>(A + m * p.sam + k * p.sak, p.sak, k, p.K, a_vec, a[r]);
            } else {
#pragma unroll
                for (int u = 0; u < V; ++u) a[r][u] = T(0);
            }
        }
        T part[P];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            T b[V];
#pragma unroll
            for (int q = 0; q < V / Vec16<T>::W; ++q) {
                typename Vec16<T>::type v =
                    *reinterpret_cast<const typename Vec16<T>::type *>(&Bs[j * LDB + lane * V + q * Vec16<T>::W]);
                const T *e = reinterpret_cast<const T *>(&v);
#pragma unroll
                for (int u = 0; u < Vec16<T>::W; ++u) b[q * Vec16<T>::W + u] = e[u];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                T x[V];
#pragma unroll
                for (int u = 0; u < V; ++u) x[u] = (k + u < p.K) ? a[r][u] * b[u] : T(-0.0);
                part[r * NJ + j] = tree_v<T, V>(x);
            }
        }
        // reduce-scatter over the P outputs
#pragma unroll
        for (int st = 0, cnt = P; cnt > 1; ++st, cnt >>= 1) {
            const int msk = 1 << st;
            const bool bit = (lane >> st) & 1;
#pragma unroll
            for (int q = 0; q < cnt / 2; ++q) {
                const T lo = part[2 * q], hi = part[2 * q + 1];
                const T send = bit ? lo : hi;
                const T keep = bit ? hi : lo;
                part[q] = keep + shfl_xor(send, msk);
            }
        }
        T x = part[0];
#pragma unroll
        for (int msk = P; msk < 64; msk <<= 1) x = x + shfl_xor(x, msk);
        carry_push<T, MAXD>(lvl, s, x);
    }
    const int o = lane % P;
    if (lane < P) {
        const int64_t m = m_base + o / NJ, n = n0 + o % NJ;
        if (m < p.M && n < p.N) {
            T *C = static_cast<T *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
            C[m * p.scm + n * p.scn] = gemm_epilogue<T>(carry_total<T, MAXD>(lvl, nseg), p, z0, z1, m, n);
        }
    }
}

// ---------------------------------------------------------------- column panel
// Narrow products (N <= 64, after swapping the operand roles when M is the
// narrow side: c^T = b^T a^T has the same products in the same K order).
// Lane l of every wave owns output column l and each wave owns RM rows, so
// the A value of a product is the same for the whole wave. Per chunk of KC
// leaves the workgroup stages, one chunk ahead (double buffered in LDS), the
// A tile [RM*WAVES rows x KC] and the B panel [KC x 64 columns] with
// coalesced loads; a wave then reads its A values as wave-uniform
// (broadcast) LDS loads and B with one 64-lane load per pair of leaves,
// shared by its RM products of each leaf. Operands of the next leaf pair are
// read while the current pair computes.
//
// Each output streams its leaves in order through a static KC-leaf tree
// (the unrolled leaf index fixes every join at compile time) and the chunk
// totals through a carry stack of depth D whose branches are wave-uniform.
// A workgroup covers one aligned power-of-two block of kpart leaves
// (blockIdx.y); the canonical tree over K equals the full tree over K
// padded with -0.0, which is the full tree over those block totals, so with
// more than one block the totals go to a workspace and tree_combine_kernel
// joins them in tree order.
// Carry-stack depth of the block-total join: up to 2^16 - 1 totals, i.e.
// K up to 2^16 - 1 blocks of 512 leaves (the totals run along grid y,
// whose limit is the same 65535).
constexpr int kCombineLevels = 16;
constexpr int64_t kMaxParts = (int64_t(1) << kCombineLevels) - 1;

struct PanelView {
    const void *a, *b;
    int64_t M, N, K;
    int64_t sam, sak, sbk, sbn;
    int64_t sa0, sa1, sb0, sb1;
    bool swapped;  // view (m, n) is output (n, m) of the problem
};

// Output element of view coordinates (z, m, n) through the problem's
// epilogue.
template <typename T>
__device__ inline void panel_store(const GemmProblem &p, const PanelView &v, int64_t z0, int64_t z1, int64_t m,
                                   int64_t n, T acc) {
    const int64_t om = v.swapped ? n : m, on = v.swapped ? m : n;
    T *C = static_cast<T *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
    C[om * p.scm + on * p.scn] = gemm_epilogue<T>(acc, p, z0, z1, om, on);
}

// Leaf i (compile-time after unrolling) of a static tree of 2^LV leaves; after
// the last leaf the tree's total is in lv[LV - 1].
template <typename T, int LV>
__device__ inline void static_push(T (&lv)[LV], int i, T carry) {
    bool done = false;
#pragma unroll
    for (int d = 0; d < LV; ++d) {
        if (!done) {
            if ((i >> d) & 1) {
                carry = lv[d] + carry;
            } else {
                lv[d] = carry;
                done = true;
            }
        }
    }
    if (!done) lv[LV - 1] = carry;
}

template <typename T>
struct Pair;
template <>
struct Pair<float> {
    typedef float type __attribute__((ext_vector_type(2)));
};
template <>
struct Pair<double> {
    typedef double type __attribute__((ext_vector_type(2)));
};

// One chunk of KC leaves for a wave's RM outputs: A from the wave-uniform
// tile rows r0.., B from the lane's column. TAIL chunks end at `live`
// leaves; the rest are -0.0. The operands of leaf pair i + 2 are read while
// pair i computes, so the LDS latency overlaps the arithmetic.
template <typename T, int RM, int KC, int LV, bool TAIL>
__device__ __attribute__((always_inline)) inline void panel_chunk(T (&lv)[RM][LV], const T (&Bc)[KC][64],
                                                                  const T (*Ac)[KC], int r0, int lane, int live) {
    using P2 = typename Pair<T>::type;
    T b[2], bn[2];
    P2 a[RM], an[RM];
    b[0] = Bc[0][lane], b[1] = Bc[1][lane];
#pragma unroll
    for (int r = 0; r < RM; ++r) a[r] = *reinterpret_cast<const P2 *>(&Ac[r0 + r][0]);
#pragma unroll
    for (int i = 0; i < KC; i += 2) {
        if (i + 2 < KC) {
            bn[0] = Bc[i + 2][lane], bn[1] = Bc[i + 3][lane];
#pragma unroll
            for (int r = 0; r < RM; ++r) an[r] = *reinterpret_cast<const P2 *>(&Ac[r0 + r][i + 2]);
        }
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            T x0 = a[r][0] * b[0], x1 = a[r][1] * b[1];
            if constexpr (TAIL) {
                if (i >= live) x0 = T(-0.0);
                if (i + 1 >= live) x1 = T(-0.0);
            }
            static_push<T, LV>(lv[r], i, x0);
            static_push<T, LV>(lv[r], i + 1, x1);
        }
        if (i + 2 < KC) {
            b[0] = bn[0], b[1] = bn[1];
#pragma unroll
            for (int r = 0; r < RM; ++r) a[r] = an[r];
        }
    }
}

template <typename T, int RM, int WAVES, int KC, int D, bool PARTIAL, bool AVEC>
__global__ __launch_bounds__(64 * WAVES) void tree_panel_kernel(PanelView v, GemmProblem p, int64_t kpart,
                                                                 T *__restrict__ part) {
    constexpr int LV = __builtin_ctz(KC);
    constexpr int ROWS = RM * WAVES;
    constexpr int BPER = KC / WAVES;                // B elements staged per thread
    constexpr int APER = ROWS * KC / (64 * WAVES);  // A elements staged per thread (a contiguous run)
    static_assert((KC & (KC - 1)) == 0 && KC % WAVES == 0 && APER == 2, "chunk shape");
    using P2 = typename Pair<T>::type;
    __shared__ T Bs[2][KC][64];
    __shared__ __attribute__((aligned(16))) T As[2][ROWS][KC];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t z = blockIdx.z, z0 = z / p.nb1, z1 = z % p.nb1;
    const int64_t mg = (int64_t)blockIdx.x * ROWS;  // first row of the workgroup
    const int64_t k_lo = (int64_t)blockIdx.y * kpart;
    const int64_t k_hi = k_lo + kpart < v.K ? k_lo + kpart : v.K;
    const int64_t nchunk = (k_hi - k_lo + KC - 1) / KC;
    const T *A = static_cast<const T *>(v.a) + z0 * v.sa0 + z1 * v.sa1;
    const T *B = static_cast<const T *>(v.b) + z0 * v.sb0 + z1 * v.sb1;
    const bool col_ok = lane < v.N;
    // this thread's A run: tile row ar, leaves ac, ac + 1
    const int ar = tid / (KC / APER), ac = (tid % (KC / APER)) * APER;
    const bool arow_ok = mg + ar < v.M;
    const T *Arow = A + (arow_ok ? mg + ar : 0) * v.sam;

    T sb[BPER], sa[APER];
    auto fetch = [&](int64_t kc) {
#pragma unroll
        for (int j = 0; j < BPER; ++j) {
            const int64_t k = kc + wave + WAVES * j;
            sb[j] = (k < k_hi && col_ok) ? B[k * v.sbk + lane * v.sbn] : T(0);
        }
        const int64_t k = kc + ac;
        if (AVEC && arow_ok && k + APER <= k_hi) {
            const P2 q = *reinterpret_cast<const P2 *>(Arow + k);
            sa[0] = q[0], sa[1] = q[1];
        } else {
#pragma unroll
            for (int u = 0; u < APER; ++u) sa[u] = (arow_ok && k + u < k_hi) ? Arow[(k + u) * v.sak] : T(0);
        }
    };
    auto put = [&](int buf) {
#pragma unroll
        for (int j = 0; j < BPER; ++j) Bs[buf][wave + WAVES * j][lane] = sb[j];
        P2 q;
        q[0] = sa[0], q[1] = sa[1];
        *reinterpret_cast<P2 *>(&As[buf][ar][ac]) = q;
    };
    fetch(k_lo);
    put(0);
    __syncthreads();

    T lvl[RM][D];
    for (int64_t c = 0; c < nchunk; ++c) {
        const int buf = (int)(c & 1);
        const int64_t kc = k_lo + c * KC;
        if (c + 1 < nchunk) fetch(kc + KC);
        T lv[RM][LV];
        if (kc + KC <= k_hi)
            panel_chunk<T, RM, KC, LV, false>(lv, Bs[buf], As[buf], wave * RM, lane, 0);
        else  // the last, partial chunk: leaves at k >= k_hi are -0.0
            panel_chunk<T, RM, KC, LV, true>(lv, Bs[buf], As[buf], wave * RM, lane, (int)(k_hi - kc));
        // chunk totals into the carry stacks: the chunk index is wave-uniform,
        // so each level is one uniform branch for all RM outputs
        const int t = __builtin_ctzll(~(unsigned long long)c);
        T carry[RM];
#pragma unroll
        for (int r = 0; r < RM; ++r) carry[r] = lv[r][LV - 1];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (d < t) {
#pragma unroll
                for (int r = 0; r < RM; ++r) carry[r] = lvl[r][d] + carry[r];
            } else if (d == t) {
#pragma unroll
                for (int r = 0; r < RM; ++r) lvl[r][d] = carry[r];
            }
        }
        // the other buffer was last read in chunk c - 1, before the barrier
        // that closed it
        if (c + 1 < nchunk) put(buf ^ 1);
        __syncthreads();
    }
    if (!col_ok) return;
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        const int64_t m = mg + wave * RM + r;
        if (m >= v.M) break;
        T total = T(0);
        bool found = false;
#pragma unroll
        for (int d = 0; d < D; ++d)
            if ((nchunk >> d) & 1) {
                total = found ? lvl[r][d] + total : lvl[r][d];
                found = true;
            }
        if constexpr (PARTIAL) {
            part[(((int64_t)blockIdx.y * gridDim.z + z) * v.M + m) * 64 + lane] = total;
        } else {
            panel_store<T>(p, v, z0, z1, m, lane, total);
        }
    }
}

// Column panel with the A leaves in scalar registers. A wave's RM rows are
// wave-uniform, so with K-contiguous A their leaves are read through the
// scalar cache (constant address space loads: A is read-only here) and
// enter the multiplies as SGPR operands; only B, one value per lane, is
// staged in LDS. Staged in LDS, every A value was a 64-lane broadcast read
// and the LDS return path, not the arithmetic, bounded the panel. The
// leaf order, padding and carry stack are tree_panel_kernel's.
template <typename T, int RM, int KC, int LV, bool TAIL, typename CT>
__device__ __attribute__((always_inline)) inline void panel_chunk_s(T (&lv)[RM][LV], const T (&Bc)[KC][64],
                                                                    CT *const (&arow)[RM], int64_t kc, int lane,
                                                                    int live) {
    T b[2], bn[2];
    b[0] = Bc[0][lane], b[1] = Bc[1][lane];
#pragma unroll
    for (int i = 0; i < KC; i += 2) {
        if (i + 2 < KC) bn[0] = Bc[i + 2][lane], bn[1] = Bc[i + 3][lane];
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            // a leaf past the live ones reads leaf kc (in range) and is replaced by -0.0
            const int64_t k0 = kc + ((TAIL && i >= live) ? 0 : i);
            const int64_t k1 = kc + ((TAIL && i + 1 >= live) ? 0 : i + 1);
            T x0 = arow[r][k0] * b[0], x1 = arow[r][k1] * b[1];
            if constexpr (TAIL) {
                if (i >= live) x0 = T(-0.0);
                if (i + 1 >= live) x1 = T(-0.0);
            }
            static_push<T, LV>(lv[r], i, x0);
            static_push<T, LV>(lv[r], i + 1, x1);
        }
        if (i + 2 < KC) b[0] = bn[0], b[1] = bn[1];
    }
}

template <typename T, int RM, int WAVES, int KC, int D, bool PARTIAL>
__global__ __launch_bounds__(64 * WAVES) void tree_panel_s_kernel(PanelView v, GemmProblem p, int64_t kpart,
                                                                   T *__restrict__ part) {
    typedef __attribute__((address_space(4))) const T CT;
    constexpr int LV = __builtin_ctz(KC);
    constexpr int ROWS = RM * WAVES;
    constexpr int BPER = KC / WAVES;  // B elements staged per thread
    static_assert((KC & (KC - 1)) == 0 && KC % WAVES == 0, "chunk shape");
    __shared__ T Bs[2][KC][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t z = blockIdx.z, z0 = z / p.nb1, z1 = z % p.nb1;
    const int64_t mg = (int64_t)blockIdx.x * ROWS;  // first row of the workgroup
    const int64_t k_lo = (int64_t)blockIdx.y * kpart;
    const int64_t k_hi = k_lo + kpart < v.K ? k_lo + kpart : v.K;
    const int64_t nchunk = (k_hi - k_lo + KC - 1) / KC;
    const T *A = static_cast<const T *>(v.a) + z0 * v.sa0 + z1 * v.sa1;
    const T *B = static_cast<const T *>(v.b) + z0 * v.sb0 + z1 * v.sb1;
    const bool col_ok = lane < v.N;
    // the wave's rows; a row past M reads row M - 1 and stores nothing
    CT *arow[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        const int64_t m = mg + wave * RM + r;
        // a global address is also its constant address space address
        arow[r] = (CT *)(uintptr_t)(A + (m < v.M ? m : v.M - 1) * v.sam);
    }

    T sb[BPER];
    auto fetch = [&](int64_t kc) {
#pragma unroll
        for (int j = 0; j < BPER; ++j) {
            const int64_t k = kc + wave + WAVES * j;
            sb[j] = (k < k_hi && col_ok) ? B[k * v.sbk + lane * v.sbn] : T(0);
        }
    };
    auto put = [&](int buf) {
#pragma unroll
        for (int j = 0; j < BPER; ++j) Bs[buf][wave + WAVES * j][lane] = sb[j];
    };
    fetch(k_lo);
    put(0);
    __syncthreads();

    T lvl[RM][D];
    for (int64_t c = 0; c < nchunk; ++c) {
        const int buf = (int)(c & 1);
        const int64_t kc = k_lo + c * KC;
        if (c + 1 < nchunk) fetch(kc + KC);
        T lv[RM][LV];
        if (kc + KC <= k_hi)
            panel_chunk_s<T, RM, KC, LV, false>(lv, Bs[buf], arow, kc, lane, KC);
        else  // the last, partial chunk: leaves at k >= k_hi are -0.0
            panel_chunk_s<T, RM, KC, LV, true>(lv, Bs[buf], arow, kc, lane, (int)(k_hi - kc));
        const int t = __builtin_ctzll(~(unsigned long long)c);
        T carry[RM];
#pragma unroll
        for (int r = 0; r < RM; ++r) carry[r] = lv[r][LV - 1];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (d < t) {
#pragma unroll
                for (int r = 0; r < RM; ++r) carry[r] = lvl[r][d] + carry[r];
            } else if (d == t) {
#pragma unroll
                for (int r = 0; r < RM; ++r) lvl[r][d] = carry[r];
            }
        }
        if (c + 1 < nchunk) put(buf ^ 1);
        __syncthreads();
    }
    if (!col_ok) return;
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        const int64_t m = mg + wave * RM + r;
        if (m >= v.M) break;
        T total = T(0);
        bool found = false;
#pragma unroll
        for (int d = 0; d < D; ++d)
            if ((nchunk >> d) & 1) {
                total = found ? lvl[r][d] + total : lvl[r][d];
                found = true;
            }
        if constexpr (PARTIAL) {
            part[(((int64_t)blockIdx.y * gridDim.z + z) * v.M + m) * 64 + lane] = total;
        } else {
            panel_store<T>(p, v, z0, z1, m, lane, total);
        }
    }
}

// Join the per-block totals of tree_panel_kernel: the canonical tree over
// the nparts block totals (adjacent pairs, odd one carried; a carry stack
// of kCombineLevels levels holds up to 2^kCombineLevels - 1 totals), then
// the epilogue. One thread per output.
template <typename T>
__global__ __launch_bounds__(256) void tree_combine_kernel(PanelView v, GemmProblem p, const T *__restrict__ part,
                                                           int64_t nparts, int64_t nz) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_z = v.M * 64;
    if (idx >= nz * per_z) return;
    const int64_t n = idx % 64;
    if (n >= v.N) return;
    const int64_t z = idx / per_z, m = (idx / 64) % v.M;
    T lvl[kCombineLevels];
    // eight block totals are read before any is pushed: one memory latency
    // per eight parts
    for (int64_t j0 = 0; j0 < nparts; j0 += 8) {
        T q[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) q[u] = j0 + u < nparts ? part[(j0 + u) * nz * per_z + idx] : T(0);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t j = j0 + u;
            if (j >= nparts) break;
            T carry = q[u];
            bool done = false;
#pragma unroll
            for (int d = 0; d < kCombineLevels; ++d) {
                if (!done) {
                    if ((j >> d) & 1) {
                        carry = lvl[d] + carry;
                    } else {
                        lvl[d] = carry;
                        done = true;
                    }
                }
            }
        }
    }
    T total = T(0);
    bool found = false;
#pragma unroll
    for (int d = 0; d < kCombineLevels; ++d)
        if ((nparts >> d) & 1) {
            total = found ? lvl[d] + total : lvl[d];
            found = true;
        }
    panel_store<T>(p, v, z / p.nb1, z % p.nb1, m, n, total);
}

// The same join for few outputs with many block totals: one wave per
// output, total j in lane j % 64 of segment j / 64 (-0.0 past nparts, at
// most four segments), each segment joined by the wave tree, then the
// segments in order. That is the full tree over the totals padded to 256
// with -0.0, i.e. their canonical tree: the same bits as the thread form.
template <typename T>
__global__ __launch_bounds__(256) void tree_combine_wave_kernel(PanelView v, GemmProblem p,
                                                                const T *__restrict__ part, int64_t nparts,
                                                                int64_t nz) {
    const int lane = threadIdx.x & 63;
    const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= nz * v.M * v.N) return;  // whole waves leave together
    const int64_t n = w % v.N, zm = w / v.N, m = zm % v.M, z = zm / v.M;
    const int64_t per_z = v.M * 64, idx = (z * v.M + m) * 64 + n;
    T seg[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int64_t j = s * 64 + lane;
        seg[s] = wave_tree_sum(j < nparts ? part[j * nz * per_z + idx] : T(-0.0));
    }
    const T total = (seg[0] + seg[1]) + (seg[2] + seg[3]);
    if (lane == 0) panel_store<T>(p, v, z / p.nb1, z % p.nb1, m, n, total);
}

// ---------------------------------------------------------------- thread per output
// Short K (<= 32): one thread per output, n fastest so B and C accesses
// coalesce. The K leaves are padded with -0.0 to P = 2^ceil(log2 K) and
// summed as a complete register tree: x + (-0.0) = x for every x, so this is
// the canonical tree over the K leaves. All loads are issued before the
// first sum (one memory latency per output, not one per leaf); AV/BV read
// a run along K with 16-byte vectors.
template <typename T, int P, bool AV, bool BV>
__global__ __launch_bounds__(256) void tree_thread_kernel(GemmProblem p, int64_t outputs) {
    constexpr int W = (int)Vec16<T>::W;
    const int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (w >= outputs) return;
    const int64_t n = w % p.N, mz = w / p.N, m = mz % p.M, z = mz / p.M;
    const int64_t z0 = z / p.nb1, z1 = z % p.nb1;
    const T *A = static_cast<const T *>(p.a) + z0 * p.sa0 + z1 * p.sa1 + m * p.sam;
    const T *B = static_cast<const T *>(p.b) + z0 * p.sb0 + z1 * p.sb1 + n * p.sbn;
    const int K = (int)p.K;
    T a[P], b[P];
#pragma unroll
    for (int k0 = 0; k0 < P; k0 += W) {
        if (AV && P >= W && k0 + W <= K) {
            const typename Vec16<T>::type v = *reinterpret_cast<const typename Vec16<T>::type *>(A + k0);
            const T *ve = reinterpret_cast<const T *>(&v);
#pragma unroll
            for (int u = 0; u < W && u < P; ++u) a[k0 + u] = ve[u];
        } else {
#pragma unroll
            for (int u = 0; u < W && k0 + u < P; ++u) a[k0 + u] = k0 + u < K ? A[(k0 + u) * p.sak] : T(0);
        }
        if (BV && P >= W && k0 + W <= K) {
            const typename Vec16<T>::type v = *reinterpret_cast<const typename Vec16<T>::type *>(B + k0);
            const T *ve = reinterpret_cast<const T *>(&v);
#pragma unroll
            for (int u = 0; u < W && u < P; ++u) b[k0 + u] = ve[u];
        } else {
#pragma unroll
            for (int u = 0; u < W && k0 + u < P; ++u) b[k0 + u] = k0 + u < K ? B[(k0 + u) * p.sbk] : T(0);
        }
    }
#pragma unroll
    for (int k = 0; k < P; ++k) a[k] = k < K ? a[k] * b[k] : T(-0.0);
#pragma unroll
    for (int s = 1; s < P; s <<= 1)
#pragma unroll
        for (int i = 0; i + s < P; i += 2 * s) a[i] = a[i] + a[i + s];
    // the empty contraction is +0
    const T total = K == 0 ? T(0) : a[0];
    T *C = static_cast<T *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
    C[m * p.scm + n * p.scn] = gemm_epilogue<T>(total, p, z0, z1, m, n);
}

bool aligned16(const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

template <typename T>
int32_t run_wave(const GemmProblem &p, hipStream_t st) {
    constexpr int V = 8;
    const int64_t outputs = p.M * p.N * p.nb0 * p.nb1;
    const bool ak = p.sak == 1 || p.K == 1, bk = p.sbk == 1 || p.K == 1;
    constexpr int64_t W = Vec16<T>::W;
    const bool av = ak && aligned16(p.a) && p.sam % W == 0 && p.sa0 % W == 0 && p.sa1 % W == 0;
    const bool bv = bk && aligned16(p.b) && p.sbn % W == 0 && p.sb0 % W == 0 && p.sb1 % W == 0;
    const int64_t blocks = (outputs + 3) / 4;
    if (!grid_fits(blocks, 256)) return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: too many outputs");
    // carry depth: DEPTH levels hold up to 2^(DEPTH - 1) segments (the last
    // push of 2^d segments lands in level d), so 9 levels cover K up to
    // 256 * 64 * V
    const bool shallow = (p.K + 64 * V - 1) / (64 * V) <= (int64_t(1) << 8);
#define CHELIS_WAVE(A_, B_)                                                                                \
    do {                                                                                                    \
        if (shallow) tree_wave_kernel<T, V, A_, B_, 9><<<(unsigned)blocks, 256, 0, st>>>(p, outputs, av, bv);    \
        else tree_wave_kernel<T, V, A_, B_, MAXD><<<(unsigned)blocks, 256, 0, st>>>(p, outputs, av, bv);         \
    } while (0)
    if (ak && bk) CHELIS_WAVE(true, true);
    else if (ak) CHELIS_WAVE(true, false);
    else if (bk) CHELIS_WAVE(false, true);
    else CHELIS_WAVE(false, false);
#undef CHELIS_WAVE
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

template <typename T>
int32_t run_tiled(const GemmProblem &p, hipStream_t st) {
    constexpr int V = sizeof(T) == 4 ? 8 : 4, R = 4, NJ = 16, WAVES = 8;
    constexpr int64_t W = Vec16<T>::W;
    const bool ak = p.sak == 1 || p.K == 1;
    const bool av = ak && aligned16(p.a) && p.sam % W == 0 && p.sa0 % W == 0 && p.sa1 % W == 0;
    const bool kfast = p.sbk == 1 || (p.sbn != 1 && p.sbk < p.sbn);
    const int64_t gx = (p.M + WAVES * R - 1) / (WAVES * R), gy = (p.N + NJ - 1) / NJ, gz = p.nb0 * p.nb1;
    if (!grid_fits(gx, 64 * WAVES) || gy > 65535 || gz > 65535)
        return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: grid too large");
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)gz);
    if (ak && kfast) tree_tiled_kernel<T, V, R, NJ, WAVES, true, true><<<grid, 64 * WAVES, 0, st>>>(p, av);
    else if (ak) tree_tiled_kernel<T, V, R, NJ, WAVES, true, false><<<grid, 64 * WAVES, 0, st>>>(p, av);
    else if (kfast) tree_tiled_kernel<T, V, R, NJ, WAVES, false, true><<<grid, 64 * WAVES, 0, st>>>(p, av);
    else tree_tiled_kernel<T, V, R, NJ, WAVES, false, false><<<grid, 64 * WAVES, 0, st>>>(p, av);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

// Column-panel launch: RM = 4 rows per wave, 4 waves, KC = 32 leaves per
// chunk, D = 5 carry levels (a block of up to 2^(D-1) = 16 chunks, 512
// leaves, leaves its total in level D - 1). The K block size shrinks
// (powers of two, >= KC) until the grid holds about four workgroups per CU;
// the block totals are joined by tree_combine_kernel. Measured on the MLP's
// narrow products: the extra workgroups outweigh the combine pass even for
// products of a few million terms (one deep block per row group is slower).
template <typename T, int D>
int32_t launch_panel(const GemmProblem &p, const PanelView &v, bool cut, hipStream_t st) {
    constexpr int RM = 4, WAVES = 4, KC = 32;
    const int64_t nz = p.nb0 * p.nb1;
    const int64_t gx = (v.M + RM * WAVES - 1) / (RM * WAVES);
    int64_t p2 = KC;
    while (p2 < v.K) p2 <<= 1;
    int64_t kpart = std::min<int64_t>(p2, (int64_t)KC << (D - 1));
    const int64_t want = 4 * (int64_t)std::max(device_cus(), 1);
    // (cutting stops at 255 block totals; a long K keeps the full block
    // and may leave up to kMaxParts)
    while (cut && kpart > KC && gx * nz * ((v.K + kpart - 1) / kpart) < want &&
           (v.K + kpart / 2 - 1) / (kpart / 2) <= 255)
        kpart >>= 1;
    const int64_t nparts = (v.K + kpart - 1) / kpart;
    if (!grid_fits(gx, 64 * WAVES) || nparts > kMaxParts || nz > 65535 ||
        !grid_fits(grid_for(nz * v.M * 64, 256), 256))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: panel grid too large");
    const dim3 grid((unsigned)gx, (unsigned)nparts, (unsigned)nz);
    // A runs load as one 2-element vector: unit K stride, aligned rows
    const bool avec = v.sak == 1 && (reinterpret_cast<uintptr_t>(v.a) % (2 * sizeof(T))) == 0 && v.sam % 2 == 0 &&
                      v.sa0 % 2 == 0 && v.sa1 % 2 == 0;
    T *ws = nullptr;
    const size_t ws_bytes = (size_t)nparts * nz * v.M * 64 * sizeof(T);
    if (nparts > 1 && !(ws = static_cast<T *>(scratch_alloc(ws_bytes))))
        return set_error(CHELIS_HIP_EHIP, "matmul: scratch allocation failed");
    // K-contiguous A: its leaves through the scalar cache
    const bool ascalar = v.sak == 1;
    if (nparts == 1) {
        if (ascalar) tree_panel_s_kernel<T, RM, WAVES, KC, D, false><<<grid, 64 * WAVES, 0, st>>>(v, p, kpart, ws);
        else if (avec) tree_panel_kernel<T, RM, WAVES, KC, D, false, true><<<grid, 64 * WAVES, 0, st>>>(v, p, kpart, ws);
        else tree_panel_kernel<T, RM, WAVES, KC, D, false, false><<<grid, 64 * WAVES, 0, st>>>(v, p, kpart, ws);
    } else {
        if (ascalar) tree_panel_s_kernel<T, RM, WAVES, KC, D, true><<<grid, 64 * WAVES, 0, st>>>(v, p, kpart, ws);
        else if (avec) tree_panel_kernel<T, RM, WAVES, KC, D, true, true><<<grid, 64 * WAVES, 0, st>>>(v, p, kpart, ws);
        else tree_panel_kernel<T, RM, WAVES, KC, D, true, false><<<grid, 64 * WAVES, 0, st>>>(v, p, kpart, ws);
    }
    hipError_t le = hipGetLastError();
    if (le == hipSuccess && nparts > 1) {
        // many totals for few outputs: lanes over the totals (a thread per
        // output would read its totals one batch after another)
        const int64_t outputs = nz * v.M * v.N;
        if (nparts >= 32 && nparts <= 256 && outputs <= 65536)
            tree_combine_wave_kernel<T><<<grid_for(outputs, 4), 256, 0, st>>>(v, p, ws, nparts, nz);
        else
            tree_combine_kernel<T><<<grid_for(nz * v.M * 64, 256), 256, 0, st>>>(v, p, ws, nparts, nz);
        le = hipGetLastError();
    }
    scratch_free(ws, ws_bytes);
    if (le != hipSuccess) return set_error(CHELIS_HIP_EHIP, "kernel launch: %s", hipGetErrorString(le));
    return CHELIS_HIP_OK;
}

template <typename T>
int32_t run_panel(const GemmProblem &p, hipStream_t st) {
    PanelView v{};
    // the narrow side goes on the lanes; a matrix-vector product (N = 1)
    // puts its outputs there instead
    v.swapped = p.N > 64 || (p.N == 1 && p.M > 1);
    if (!v.swapped) {
        v.a = p.a, v.b = p.b, v.M = p.M, v.N = p.N, v.sam = p.sam, v.sak = p.sak, v.sbk = p.sbk, v.sbn = p.sbn;
        v.sa0 = p.sa0, v.sa1 = p.sa1, v.sb0 = p.sb0, v.sb1 = p.sb1;
    } else {
        v.a = p.b, v.b = p.a, v.M = p.N, v.N = p.M, v.sam = p.sbn, v.sak = p.sbk, v.sbk = p.sak, v.sbn = p.sam;
        v.sa0 = p.sb0, v.sa1 = p.sb1, v.sb0 = p.sa0, v.sb1 = p.sa1;
    }
    v.K = p.K;
    if (v.N > 64) return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: panel kernel needs min(M, N) <= 64");
    return launch_panel<T, 5>(p, v, true, st);
}

template <typename T, int P>
void launch_thread(const GemmProblem &p, int64_t outputs, bool av, bool bv, hipStream_t st) {
    const unsigned blocks = (unsigned)((outputs + 255) / 256);
    if (av && bv) tree_thread_kernel<T, P, true, true><<<blocks, 256, 0, st>>>(p, outputs);
    else if (av) tree_thread_kernel<T, P, true, false><<<blocks, 256, 0, st>>>(p, outputs);
    else if (bv) tree_thread_kernel<T, P, false, true><<<blocks, 256, 0, st>>>(p, outputs);
    else tree_thread_kernel<T, P, false, false><<<blocks, 256, 0, st>>>(p, outputs);
}

template <typename T>
int32_t run_thread(const GemmProblem &p, hipStream_t st) {
    if (p.K > 32) return set_error(CHELIS_HIP_EDOMAIN, "matmul: short-K kernel holds K <= 32");
    const int64_t outputs = p.M * p.N * p.nb0 * p.nb1;
    const int64_t blocks = (outputs + 255) / 256;
    if (!grid_fits(blocks, 256)) return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: too many outputs");
    constexpr int64_t W = Vec16<T>::W;
    // a vector read of A (B) needs K contiguous and every row (column) start 16-byte aligned
    const bool av = p.sak == 1 && aligned16(p.a) && (p.sam % W == 0 || p.M == 1) && p.sa0 % W == 0 && p.sa1 % W == 0;
    const bool bv = p.sbk == 1 && aligned16(p.b) && (p.sbn % W == 0 || p.N == 1) && p.sb0 % W == 0 && p.sb1 % W == 0;
    if (p.K <= 1) launch_thread<T, 1>(p, outputs, false, false, st);
    else if (p.K <= 2) launch_thread<T, 2>(p, outputs, false, false, st);
    else if (p.K <= 4) launch_thread<T, 4>(p, outputs, av, bv, st);
    else if (p.K <= 8) launch_thread<T, 8>(p, outputs, av, bv, st);
    else if (p.K <= 16) launch_thread<T, 16>(p, outputs, av, bv, st);
    else launch_thread<T, 32>(p, outputs, av, bv, st);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

}  // namespace

int32_t gemm_tree_wave(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    return dt == CHELIS_DTYPE_F32 ? run_wave<float>(p, st) : run_wave<double>(p, st);
}
int32_t gemm_tree_tiled(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    return dt == CHELIS_DTYPE_F32 ? run_tiled<float>(p, st) : run_tiled<double>(p, st);
}
int32_t gemm_tree_panel(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    return dt == CHELIS_DTYPE_F32 ? run_panel<float>(p, st) : run_panel<double>(p, st);
}
int32_t gemm_tree_thread(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    return dt == CHELIS_DTYPE_F32 ? run_thread<float>(p, st) : run_thread<double>(p, st);
}

}  // namespace chelis

// Dense matmul on the CDNA4 matrix cores, and the matmul / linear entry
// points with their shape dispatch.
//
// MFMA tile kernel. A 256-thread workgroup (4 waves, 2 x 2) owns a 128 x 128
// tile of C; each wave owns 64 x 64 = 4 x 4 blocks of 16 x 16, accumulated
// by v_mfma_f32_16x16x4_f32 (f32) or v_mfma_f64_16x16x4_f64 (f64); a 64 x 64
// tile (32 x 32 per wave) serves products with few 128-tiles. K moves in
// steps of BK (16 for f32, 8 for f64; twice that for the 64-tile) through
// two LDS buffers: while the
// matrix cores consume one buffer, the next A and B tiles are already in
// flight from HBM into registers and land in the other buffer after the
// step, so there is one barrier per K step.
//
// LDS holds both operands K-contiguous (As[m][k], Bs[n][k]) with the row
// padded by 16 bytes (80 or 144 bytes). An MFMA of shape 16x16x4 takes A[i][q] from lane
// q*16 + i and B[q][j] from lane q*16 + j, and returns C[i][j] in lane
// q*16 + j, item r, with i = 4q + r for f32 and i = q + 4r for f64 (both
// checked on gfx950 with a one-wave layout probe). Over the KV = BK/4 MFMAs of one
// step, lane group q supplies k = q*KV + t for MFMA t, so both fragments of
// a lane are KV consecutive k values: one or two 16-byte LDS reads each,
// and the padded row pitch puts the 8 rows a read phase touches on 8
// disjoint 4-bank groups.
//
// Operands are strided views (a transposed operand is a stride swap):
// each one is staged with 16-byte vector loads along whichever of its axes
// is contiguous (K or the outer axis), or element by element when neither
// is.
//
// Blocks are numbered so that each of the 8 XCDs (workgroups are dealt to
// XCDs round-robin) receives one contiguous run of tiles, walked in groups
// of 8 tile-rows, so the A row-panels and B column-panels a tile reads are
// shared inside that XCD's L2.
#include "gemm.h"

#include <type_traits>

namespace chelis {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;
template <>
struct Mfma<float> {
    using acc_t = f32x4;
    static constexpr int V = 4;
    // accumulator item r of lane group q holds row 4q + r of the 16x16 block
    __device__ static int row(int q, int r) { return 4 * q + r; }
    __device__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma<double> {
    using acc_t = f64x4;
    static constexpr int V = 2;
    // accumulator item r of lane group q holds row q + 4r of the 16x16 block
    __device__ static int row(int q, int r) { return q + 4 * r; }
    __device__ static acc_t step(double a, double b, acc_t c) {
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
    }
};

constexpr int THREADS = 256;

// K depth of one step. The 128-tile takes 16 (f32) / 8 (f64): four MFMA
// chains of 4 x 4 blocks per wave between barriers. The 64-tile has a
// quarter of those blocks per wave, so it takes twice the depth, keeping
// the matrix work between barriers (and the lead the two register staging
// sets give each global load, two steps) at half the 128-tile's rather than
// a quarter. The LDS row pitch is BK plus 16 bytes: 80 or 144 bytes, so
// the 8 rows one 16-byte read phase touches fall on 8 disjoint 4-bank groups.
template <typename T, int TM>
struct Depth {
    static constexpr int BK = (sizeof(T) == 8 ? 8 : 16) * (TM == 2 ? 2 : 1);
    static constexpr int LD = BK + 16 / (int)sizeof(T);
    static constexpr int KV = BK / 4;  // consecutive k per lane and MFMA chain
};

template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
    using type = float4;
};
template <>
struct Vec16<double> {
    using type = double2;
};

// Layout of a staged operand: 0 = vectors along K, 1 = vectors along the
// outer axis (M of A, N of B), 2 = element by element.
template <typename T, int LAY, int ROWS, int BK_, int LD_>
struct Stage {
    static constexpr int BK = BK_, V = Mfma<T>::V, LD = LD_;
    static constexpr int NE = ROWS * BK / THREADS;  // elements per thread
    static constexpr int NV = NE / V;               // vectors per thread
    T r[NE];

    // element (row, k) lives at base[row * s_row + k * s_k]. CHECK = false:
    // the caller guarantees aligned vectors inside the operand (LAY 0 or 1),
    // so every load is an unconditional 16-byte vector load; straight-line
    // loads let the compiler wait for exactly the older ones.
    template <bool CHECK = true>
    __device__ void load(const T *__restrict__ base, int64_t s_row, int64_t s_k, int64_t row0, int64_t rows,
                         int64_t k0, int64_t K, bool vec_ok) {
        const int t = threadIdx.x;
        if constexpr (!CHECK && LAY != 2) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int idx = t + THREADS * j;
                const T *p;
                if constexpr (LAY == 0) {
                    const int row = idx / (BK / V), kv = (idx % (BK / V)) * V;
                    p = base + (row0 + row) * s_row + (k0 + kv);
                } else {
                    const int k = idx % BK, rv = (idx / BK) * V;
                    p = base + (row0 + rv) + (k0 + k) * s_k;
                }
                typename Vec16<T>::type q = *reinterpret_cast<const typename Vec16<T>::type *>(p);
                const T *qe = reinterpret_cast<const T *>(&q);
#pragma unroll
                for (int u = 0; u < V; ++u) r[j * V + u] = qe[u];
            }
        } else if constexpr (LAY == 0) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int idx = t + THREADS * j;
                const int row = idx / (BK / V), kv = (idx % (BK / V)) * V;
                const int64_t gr = row0 + row, gk = k0 + kv;
                const T *p = base + gr * s_row + gk;
                if (vec_ok && gr < rows && gk + V <= K) {
                    typename Vec16<T>::type q = *reinterpret_cast<const typename Vec16<T>::type *>(p);
                    const T *qe = reinterpret_cast<const T *>(&q);
#pragma unroll
                    for (int u = 0; u < V; ++u) r[j * V + u] = qe[u];
                } else {
#pragma unroll
                    for (int u = 0; u < V; ++u) r[j * V + u] = (gr < rows && gk + u < K) ? p[u] : T(0);
                }
            }
        } else if constexpr (LAY == 1) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int idx = t + THREADS * j;
                const int k = idx % BK, rv = (idx / BK) * V;
                const int64_t gr = row0 + rv, gk = k0 + k;
                const T *p = base + gr + gk * s_k;
                if (vec_ok && gk < K && gr + V <= rows) {
                    typename Vec16<T>::type q = *reinterpret_cast<const typename Vec16<T>::type *>(p);
                    const T *qe = reinterpret_cast<const T *>(&q);
#pragma unroll
                    for (int u = 0; u < V; ++u) r[j * V + u] = qe[u];
                } else {
#pragma unroll
                    for (int u = 0; u < V; ++u) r[j * V + u] = (gk < K && gr + u < rows) ? p[u] : T(0);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < NE; ++j) {
                const int idx = t + THREADS * j;
                const int row = idx / BK, k = idx % BK;
                const int64_t gr = row0 + row, gk = k0 + k;
                r[j] = (gr < rows && gk < K) ? base[gr * s_row + gk * s_k] : T(0);
            }
        }
    }

    __device__ void store(T *__restrict__ s) const {
        const int t = threadIdx.x;
        if constexpr (LAY == 0) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int idx = t + THREADS * j;
                const int row = idx / (BK / V), kv = (idx % (BK / V)) * V;
                typename Vec16<T>::type q;
                T *qe = reinterpret_cast<T *>(&q);
#pragma unroll
                for (int u = 0; u < V; ++u) qe[u] = r[j * V + u];
                *reinterpret_cast<typename Vec16<T>::type *>(s + row * LD + kv) = q;
            }
        } else if constexpr (LAY == 1) {
            // k fastest across lanes: each transposed store of a wave writes
            // runs of consecutive k in a few rows instead of one k in 64 rows
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int idx = t + THREADS * j;
                const int k = idx % BK, rv = (idx / BK) * V;
#pragma unroll
                for (int u = 0; u < V; ++u) s[(rv + u) * LD + k] = r[j * V + u];
            }
        } else {
#pragma unroll
            for (int j = 0; j < NE; ++j) {
                const int idx = t + THREADS * j;
                s[(idx / BK) * LD + idx % BK] = r[j];
            }
        }
    }
};

// f64 holds its 64x64 accumulators in 128 registers; capping the kernel at
// 256 registers per lane keeps two waves per SIMD resident (measured 1.6x
// over one wave at 4096^3). f32 is fastest with the compiler's own choice.
template <typename T>
constexpr int kMinWavesPerEu = sizeof(T) == 8 ? 2 : 1;

// TM = 16x16 blocks per wave and dimension: 4 gives the 128 x 128 tile for
// large products, 2 a 64 x 64 tile for products with few 128-tiles.
// Split K (kchunk > 0): grid.z slices K into runs of kchunk (a multiple of
// BK) and each slice stores its raw sums to part[slice][z][m][n]; a combine
// pass adds the slices in slice order and applies the epilogue.
template <typename T, int ALAY, int BLAY, int TM, bool GELU>
__global__ __launch_bounds__(THREADS, kMinWavesPerEu<T>) void gemm_mfma_kernel(GemmProblem p, int64_t tiles_m,
                                                                               int64_t tiles_n, bool a_vec,
                                                                               bool b_vec, T *part,
                                                                               int64_t kchunk) {
    using M = Mfma<T>;
    using acc_t = typename M::acc_t;
    using D = Depth<T, TM>;
    constexpr int BK = D::BK, LD = D::LD, KV = D::KV, V = M::V, NVF = KV / V;
    constexpr int BM = 32 * TM, BN = 32 * TM, WT = 16 * TM;
    __shared__ __attribute__((aligned(16))) T As[2][BM * LD];
    __shared__ __attribute__((aligned(16))) T Bs[2][BN * LD];

    // XCD-aware tile order.
    const int64_t tiles = tiles_m * tiles_n;
    int64_t bid = blockIdx.x;
    if (tiles % 8 == 0) bid = (bid % 8) * (tiles / 8) + bid / 8;
    constexpr int64_t GM = 8;
    const int64_t group = bid / (GM * tiles_n);
    const int64_t first = group * GM;
    const int64_t gsz = (tiles_m - first) < GM ? (tiles_m - first) : GM;
    const int64_t in_group = bid % (GM * tiles_n);
    const int64_t m0 = (first + in_group % gsz) * BM;
    const int64_t n0 = (in_group / gsz) * BN;
    // causal 1: a tile wholly above the diagonal is never read (the whole
    // workgroup leaves before any barrier); causal 2: a[m][k] = 0 for k > m
    if (p.causal == 1 && n0 > m0 + BM - 1) return;
    int64_t K = (p.causal == 2 && m0 + BM < p.K) ? m0 + BM : p.K;

    const int64_t z = blockIdx.y;
    const int64_t z0 = z / p.nb1, z1 = z % p.nb1;
    const T *A = static_cast<const T *>(p.a) + z0 * p.sa0 + z1 * p.sa1;
    const T *B = p.nbz ? static_cast<const T *>(p.bz[z]) : static_cast<const T *>(p.b) + z0 * p.sb0 + z1 * p.sb1;
    if (kchunk > 0) {
        const int64_t kb = (int64_t)blockIdx.z * kchunk;
        K = (K - kb < kchunk ? K - kb : kchunk);
        A += kb * p.sak;
        B += kb * p.sbk;
    }

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, fq = lane >> 4;

    acc_t acc[TM][TM];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = acc_t{};

    // Two register staging sets (measured: f32 4096^3 1.42 -> 1.17 ms, f64
    // 2.44 -> 2.31 ms over one; a third set gained nothing).
    Stage<T, ALAY, BM, BK, LD> sa0, sa1;
    Stage<T, BLAY, BN, BK, LD> sb0, sb1;
    const int64_t ksteps = (K + BK - 1) / BK;
    // an interior tile of aligned operands and whole K steps loads without checks
    const bool inside = a_vec && b_vec && ALAY != 2 && BLAY != 2 && m0 + BM <= p.M && n0 + BN <= p.N && K % BK == 0;

    // step ks computes from LDS buffer ks % 2; (sa_n, sb_n) hold step ks + 1
    // The body has no branches around its loads and stores: a step past the
    // last is clamped to the last, so the extra loads read valid memory and
    // the extra store fills the LDS buffer no later step reads. Straight-line
    // memory operations let the compiler wait for exactly the older loads.
    // a lane's fragments of one step: KV consecutive k, in NVF 16-byte LDS reads
    struct Frags {
        typename Vec16<T>::type a[TM][NVF], b[TM][NVF];
    };
    auto read_frags = [&](Frags &f, int buf) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int h = 0; h < NVF; ++h)
                f.a[i][h] = *reinterpret_cast<const typename Vec16<T>::type *>(
                    &As[buf][(wm * WT + i * 16 + fr) * LD + fq * KV + h * V]);
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int h = 0; h < NVF; ++h)
                f.b[j][h] = *reinterpret_cast<const typename Vec16<T>::type *>(
                    &Bs[buf][(wn * WT + j * 16 + fr) * LD + fq * KV + h * V]);
    };
    auto mfmas = [&](const Frags &f) {
#pragma unroll
        for (int t = 0; t < KV; ++t)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    acc[i][j] = M::step(reinterpret_cast<const T *>(f.a[i])[t],
                                        reinterpret_cast<const T *>(f.b[j])[t], acc[i][j]);
    };

    // 128-tiles: both LDS buffers hold a step. At the top of step s, buffer
    // s % 2 holds step s (already in this lane's registers as fragments)
    // and buffer (s + 1) % 2 step s + 1. Step s reads the fragments of step
    // s + 1 while its matrix work runs, then overwrites buffer s % 2 with
    // step s + 2 from a register staging set and refills that set from
    // memory with step s + 4; one barrier ends the step. The matrix cores
    // never wait for an LDS read after the barrier (measured: f32 4096^3
    // 1.13 -> 1.09 ms, f64 2.22 -> 2.03 ms).
    // 64-tiles (measured faster this way: 4096 x 1024 x 1024 f32 in 90
    // against 98 us): step s reads step s from buffer s % 2, runs its matrix
    // work, stores step s + 1 into the other buffer and refills that set
    // with step s + 3.
    // Either way each global load has two whole steps to arrive before its
    // LDS store, and the body has no branches around its loads and stores:
    // a step past the last is clamped to the last, so the extra loads read
    // valid memory and the extra LDS traffic touches buffers no later step
    // reads. Straight-line memory operations let the compiler wait for
    // exactly the older loads.
    auto run = [&](auto check) {
        constexpr bool CK = decltype(check)::value;
        const int64_t last = ksteps - 1;
        auto kstep = [&](int64_t s) { return (s < last ? s : last) * BK; };
        auto load = [&](Stage<T, ALAY, BM, BK, LD> &sa, Stage<T, BLAY, BN, BK, LD> &sb, int64_t s) {
            sa.template load<CK>(A, p.sam, p.sak, m0, p.M, kstep(s), K, a_vec);
            sb.template load<CK>(B, p.sbn, p.sbk, n0, p.N, kstep(s), K, b_vec);
        };
        auto store = [&](const Stage<T, ALAY, BM, BK, LD> &sa, const Stage<T, BLAY, BN, BK, LD> &sb, int buf) {
            sa.store(As[buf]);
            sb.store(Bs[buf]);
        };
        if constexpr (TM == 2) {
            load(sa0, sb0, 0);
            load(sa1, sb1, 1);
            store(sa0, sb0, 0);
            load(sa0, sb0, 2);
            __syncthreads();
            auto step = [&](int64_t s, Stage<T, ALAY, BM, BK, LD> &sa_n, Stage<T, BLAY, BN, BK, LD> &sb_n) {
                const int buf = s & 1;
                Frags f;
                read_frags(f, buf);
                mfmas(f);
                store(sa_n, sb_n, buf ^ 1);
                load(sa_n, sb_n, s + 3);
                __syncthreads();
            };
            int64_t ks = 0;
            for (; ks + 1 < ksteps; ks += 2) {
                step(ks, sa1, sb1);
                step(ks + 1, sa0, sb0);
            }
            if (ks < ksteps) step(ks, sa1, sb1);
        } else {
            load(sa0, sb0, 0);
            load(sa1, sb1, 1);
            store(sa0, sb0, 0);
            store(sa1, sb1, 1);
            load(sa0, sb0, 2);
            load(sa1, sb1, 3);
            __syncthreads();
            Frags f0, f1;
            read_frags(f0, 0);
            __syncthreads();  // every lane has step 0 before step 0 overwrites buffer 0
            auto step = [&](int64_t s, Frags &cur, Frags &next, Stage<T, ALAY, BM, BK, LD> &sa_n,
                            Stage<T, BLAY, BN, BK, LD> &sb_n) {
                const int buf = s & 1;
                read_frags(next, buf ^ 1);
                mfmas(cur);
                store(sa_n, sb_n, buf);
                load(sa_n, sb_n, s + 4);
                __syncthreads();
            };
            int64_t ks = 0;
            for (; ks + 1 < ksteps; ks += 2) {
                step(ks, f0, f1, sa0, sb0);
                step(ks + 1, f1, f0, sa1, sb1);
            }
            if (ks < ksteps) step(ks, f0, f1, sa0, sb0);
        }
    };
    if (inside) run(std::false_type{});
    else run(std::true_type{});

    if (kchunk > 0) {
        T *P = part + ((int64_t)blockIdx.z * gridDim.y + z) * p.M * p.N;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t m = m0 + wm * WT + i * 16 + M::row(fq, r);
                    const int64_t n = n0 + wn * WT + j * 16 + fr;
                    if (m < p.M && n < p.N) P[m * p.N + n] = acc[i][j][r];
                }
        return;
    }
    T *C = static_cast<T *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
    if constexpr (!GELU && sizeof(T) == 4) {
        // The tile through LDS in quarters of BM/4 rows, then each thread
        // finishes V consecutive columns of a row per step - its bias
        // elements read once, residual, output (and the loads) as 16-byte
        // vectors where the layout allows. Straight from the accumulators,
        // each lane would write 64-byte pieces of four rows per store and
        // read the bias and residual an element at a time (measured on
        // 4096 x 4096 x 1024 with a bias: 288 -> 278 us; the transformer
        // block 974 -> 959 us).
        constexpr int V = 16 / (int)sizeof(T);
        using VT = typename Vec16<T>::type;
        constexpr int QR = BM / 4, LDT = BN + V, CG = BN / V, RS = THREADS / CG;
        static_assert(QR * LDT <= 2 * BM * LD, "quarter tile fits in As");
        T *tile = &As[0][0];
        const int cg = threadIdx.x % CG, r0 = threadIdx.x / CG;
        const int64_t n = n0 + V * cg;
        const T *bias = static_cast<const T *>(p.nbz ? p.biasz[z0 * p.nb1 + z1] : p.bias);
        const T *resid = static_cast<const T *>(p.resid);
        const int64_t boff = p.nbz ? 0 : z0 * p.sbias0 + z1 * p.sbias1;
        const T *rbase = resid ? resid + z0 * p.sr0 + z1 * p.sr1 : nullptr;
        const bool vec = p.scn == 1 && p.scm % V == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0 &&
                         p.N % V == 0 &&
                         (!resid || (p.srn == 1 && p.srm % V == 0 && (reinterpret_cast<uintptr_t>(rbase) & 15) == 0));
        T b[V];
#pragma unroll
        for (int u = 0; u < V; ++u) b[u] = bias && n + u < p.N ? bias[boff + (n + u) * p.sbias] : T(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            __syncthreads();  // As: the main loop's (or the last quarter's) reads are done
            if (wm == q / 2) {
#pragma unroll
                for (int ii = 0; ii < TM / 2; ++ii)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            tile[(ii * 16 + M::row(fq, r)) * LDT + wn * WT + j * 16 + fr] =
                                acc[(q % 2) * (TM / 2) + ii][j][r];
            }
            __syncthreads();
#pragma unroll
            for (int row = r0; row < QR; row += RS) {
                const int64_t m = m0 + q * QR + row;
                if (m >= p.M) continue;
                const VT t = *reinterpret_cast<const VT *>(&tile[row * LDT + V * cg]);
                const T *tv = reinterpret_cast<const T *>(&t);
                if (vec && n < p.N) {
                    VT rv{};
                    if (resid) rv = *reinterpret_cast<const VT *>(rbase + m * p.srm + n);
                    const T *rr = reinterpret_cast<const T *>(&rv);
                    VT o;
                    T *oo = reinterpret_cast<T *>(&o);
#pragma unroll
                    for (int u = 0; u < V; ++u) oo[u] = epilogue_values<T, false>(tv[u], p, bias != nullptr, b[u], rr[u]);
                    *reinterpret_cast<VT *>(C + m * p.scm + n) = o;
                } else {
#pragma unroll
                    for (int u = 0; u < V; ++u)
                        if (n + u < p.N) {
                            const T r = resid ? rbase[m * p.srm + (n + u) * p.srn] : T(0);
                            C[m * p.scm + (n + u) * p.scn] = epilogue_values<T, false>(tv[u], p, bias != nullptr, b[u], r);
                        }
                }
            }
        }
        return;
    }
    if constexpr (GELU && sizeof(T) == 4) {
        // The GELU graph once, not once per held output: the tile goes
        // through LDS in quarters of BM/4 rows; the two waves owning a
        // quarter write their accumulators, then every thread runs the
        // epilogue over the quarter in a loop that is not unrolled, with
        // consecutive threads on consecutive columns (coalesced stores).
        // Inline per output, the graph took the kernel to one wave per SIMD
        // with spills.
        constexpr int QR = BM / 4, LDT = BN + 8;
        static_assert(QR * LDT <= 2 * BM * LD, "quarter tile fits in As");
        T *tile = &As[0][0];
        // the erfc and exp tables in LDS for the epilogue's GELU (published
        // by the first quarter's barrier)
        __shared__ ErfcLdsStore gtab;
        gtab.fill<THREADS>();
        const ErfcTablesLds tb = gtab.tabs();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            __syncthreads();  // As: the main loop's (or the last quarter's) reads are done
            if (wm == q / 2) {
#pragma unroll
                for (int ii = 0; ii < TM / 2; ++ii)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            tile[(ii * 16 + M::row(fq, r)) * LDT + wn * WT + j * 16 + fr] =
                                acc[(q % 2) * (TM / 2) + ii][j][r];
            }
            __syncthreads();
            // THREADS is a multiple of BN: each thread keeps one column, so
            // its bias element is read once, ahead of the loop
            static_assert(THREADS % BN == 0, "one column per thread");
            const int col = threadIdx.x % BN;
            const int64_t n = n0 + col;
            const T *bias = static_cast<const T *>(p.nbz ? p.biasz[z0 * p.nb1 + z1] : p.bias);
            const bool nin = n < p.N, hb = bias != nullptr;
            const T b = hb && nin ? bias[(p.nbz ? 0 : z0 * p.sbias0 + z1 * p.sbias1) + n * p.sbias] : T(0);
            const T *resid = static_cast<const T *>(p.resid);
            // four rows in flight per thread (4096 x 4096 x 1024 with the
            // GELU epilogue: 304.4 us rolled, 304.8 unrolled by 2, 300.9 by 4)
#pragma unroll 4
            for (int row = threadIdx.x / BN; row < QR; row += THREADS / BN) {
                const int64_t m = m0 + q * QR + row;
                if (m < p.M && nin) {
                    const T r = resid ? resid[z0 * p.sr0 + z1 * p.sr1 + m * p.srm + n * p.srn] : T(0);
                    C[m * p.scm + n * p.scn] = epilogue_values<T, true>(tile[row * LDT + col], p, hb, b, r, tb);
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * WT + i * 16 + M::row(fq, r);
                const int64_t n = n0 + wn * WT + j * 16 + fr;
                if (m < p.M && n < p.N)
                    C[m * p.scm + n * p.scn] = gemm_epilogue<T, GELU>(acc[i][j][r], p, z0, z1, m, n);
            }
}

// c[z][m][n] = epilogue(sum over slices s, in order, of part[s][z][m][n]).
// Four consecutive columns per thread; tpr (a power of two, at most 256)
// threads per row cover its first 4 tpr columns, 256 / tpr rows per
// workgroup, and grid y steps over further runs of 1024 columns. The slices
// are read as vectors when N is a multiple of four (each slice row then
// starts aligned), and no thread divides per element. VEC (N a multiple of
// four; output, residual and an unbatched-pointer bias contiguous along n
// and 16-byte aligned at every row): the bias, residual and output as
// vectors too.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void splitk_combine_kernel(GemmProblem p, const T *part, int ks, int64_t nz,
                                                             int tpr) {
    const int64_t row = (int64_t)blockIdx.x * (256 / tpr) + threadIdx.x / tpr;
    const int64_t n0 = (int64_t)blockIdx.y * 1024 + (threadIdx.x % tpr) * 4;
    if (row >= nz * p.M || n0 >= p.N) return;
    const int64_t z = row / p.M, m = row - z * p.M, total = nz * p.M * p.N;
    const int64_t z0 = z / p.nb1, z1 = z % p.nb1;
    const T *src = part + row * p.N + n0;
    T v[4];
    if (p.N % 4 == 0) {
        using V4 = typename std::conditional<sizeof(T) == 4, float4, double4>::type;
        V4 q = *reinterpret_cast<const V4 *>(src);
        v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
        for (int s = 1; s < ks; ++s) {
            q = *reinterpret_cast<const V4 *>(src + s * total);
            v[0] += q.x, v[1] += q.y, v[2] += q.z, v[3] += q.w;
        }
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = n0 + u < p.N ? src[u] : T(0);
        for (int s = 1; s < ks; ++s)
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] += n0 + u < p.N ? src[s * total + u] : T(0);
    }
    T *C = static_cast<T *>(p.c) + z0 * p.sc0 + z1 * p.sc1 + m * p.scm;
    if constexpr (VEC) {
        using V4 = typename std::conditional<sizeof(T) == 4, float4, double4>::type;
        const T *bias = static_cast<const T *>(p.bias);
        V4 b{}, r{};
        if (bias) b = *reinterpret_cast<const V4 *>(bias + z0 * p.sbias0 + z1 * p.sbias1 + n0);
        if (p.resid)
            r = *reinterpret_cast<const V4 *>(static_cast<const T *>(p.resid) + z0 * p.sr0 + z1 * p.sr1 + m * p.srm + n0);
        const bool hb = bias != nullptr;
        V4 o;
        o.x = epilogue_values<T>(v[0], p, hb, b.x, r.x);
        o.y = epilogue_values<T>(v[1], p, hb, b.y, r.y);
        o.z = epilogue_values<T>(v[2], p, hb, b.z, r.z);
        o.w = epilogue_values<T>(v[3], p, hb, b.w, r.w);
        *reinterpret_cast<V4 *>(C + n0) = o;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (n0 + u < p.N) C[(n0 + u) * p.scn] = gemm_epilogue<T>(v[u], p, z0, z1, m, n0 + u);
    }
}

// The vector form of splitk_combine_kernel applies: every row of the output,
// the residual and the bias starts 16-byte aligned and runs along n.
template <typename T>
bool combine_vec_ok(const GemmProblem &p, int64_t nz) {
    auto al = [](const void *q, int64_t elems) {
        return (reinterpret_cast<uintptr_t>(q) % 16) == 0 && (elems * (int64_t)sizeof(T)) % 16 == 0;
    };
    if (p.N % 4 || p.scn != 1 || !al(p.c, p.scm) || (nz > 1 && (!al(p.c, p.sc0) || !al(p.c, p.sc1)))) return false;
    if (p.resid && (p.srn != 1 || !al(p.resid, p.srm) || (nz > 1 && (!al(p.resid, p.sr0) || !al(p.resid, p.sr1)))))
        return false;
    if (p.nbz) return false;
    if (p.bias && (p.sbias != 1 || !al(p.bias, 0) || (nz > 1 && (!al(p.bias, p.sbias0) || !al(p.bias, p.sbias1)))))
        return false;
    return true;
}

template <typename T>
int lay_of(int64_t s_outer, int64_t s_k, const void *base, int64_t outer, int64_t K, bool *vec_ok) {
    constexpr int V = Mfma<T>::V;
    const bool al = (reinterpret_cast<uintptr_t>(base) & 15u) == 0;
    if (s_k == 1 || K == 1) {
        *vec_ok = al && (outer == 1 || s_outer % V == 0);
        return 0;
    }
    if (s_outer == 1 || outer == 1) {
        *vec_ok = al && s_k % V == 0;
        return 1;
    }
    *vec_ok = false;
    return 2;
}

// Occupancy of the f32 128-tile kernel without the GELU epilogue: its 40 KiB
// of LDS allow three workgroups per CU. Its registers decide first: the
// current build holds 224 per lane (116 vector + 108 accumulation), two
// waves per SIMD, so two workgroups per CU. Were the count to drop to 168 or
// fewer, a grid of T tiles would run in ceil(T / 3C) rounds of three; two
// per CU (ceil(T / 2C) rounds of two) is then kept when that is fewer
// workgroup-slots in all, e.g. 1024 tiles on 256 CUs as two full rounds of
// two rather than a round of three and a third of one (measured 1.42 ms
// against 1.54 ms at 4096^3 with an earlier build that fitted three).
// Dynamic LDS beyond a third of the CU's 160 KiB pins two.
constexpr size_t kPinTwoLds = 16384;

template <typename T, int AL, int BL, int TM>
void launch_mfma(const GemmProblem &p, dim3 grid, int64_t tm, int64_t tn, bool av, bool bv, T *part, int64_t kchunk,
                 hipStream_t st) {
    // split-K slices store raw sums: the combine pass applies the epilogue
    if (p.act == CHELIS_ACT_GELU && kchunk == 0) {
        gemm_mfma_kernel<T, AL, BL, TM, true><<<grid, THREADS, 0, st>>>(p, tm, tn, av, bv, part, kchunk);
        return;
    }
    size_t dyn = 0;
    if (sizeof(T) == 4 && TM == 4) {
        const int64_t C = device_cus(), t = (int64_t)grid.x * grid.y * grid.z;
        if (((t + 2 * C - 1) / (2 * C)) * 2 <= ((t + 3 * C - 1) / (3 * C)) * 3) dyn = kPinTwoLds;
    }
    gemm_mfma_kernel<T, AL, BL, TM, false><<<grid, THREADS, dyn, st>>>(p, tm, tn, av, bv, part, kchunk);
}

// Slices of K for a product whose tiles cannot fill the chip. 64-tiles:
// enough slices to give every CU about three workgroups (binary64; two for
// binary32), each slice at least 256 deep (128 for binary32; a shorter run
// does not amortize a tile's first loads and its store). (Measured on the skinny f64 8192 x 64 x 4096, 128 64-tiles: 4
// slices 109.5 us, 6 slices 102.5 us, 8 slices 113.5 us.) 128-tiles (chosen
// for fewer than two per CU only when K is long, see run_mfma): two
// workgroups per CU, each slice at least 1024 deep. At most 16 slices;
// returns 1 for no split.
template <typename T, int TM>
int64_t split_count(const GemmProblem &p, int64_t tiles, int64_t *kchunk) {
    constexpr int64_t BK = Depth<T, TM>::BK;
    const int64_t cus = device_cus();
    // 64-tiles, binary32: two workgroups per CU and slices down to 128 deep
    // (the MLP's 1024 x 512 x 784 product: 4 slices 15.7 us, 3 slices 18.8
    // us, 6 slices 18.5 us)
    const int64_t per_cu = TM == 2 ? (sizeof(T) == 4 ? 2 : 3) : 2;
    const int64_t min_depth = TM == 2 ? (sizeof(T) == 4 ? 128 : 256) : 1024;
    if (p.causal != 0 || tiles >= (TM == 2 ? cus : 2 * cus) || p.K < 2 * min_depth) return 1;
    int64_t ks = (per_cu * cus + tiles - 1) / tiles;
    if (ks > p.K / min_depth) ks = p.K / min_depth;
    if (ks > 16) ks = 16;
    if (ks < 2) return 1;
    int64_t kc = (p.K + ks - 1) / ks;
    kc = (kc + BK - 1) / BK * BK;
    ks = (p.K + kc - 1) / kc;
    if (ks < 2 || ks * p.nb0 * p.nb1 * p.M * p.N > (int64_t(64) << 20)) return 1;
    *kchunk = kc;
    return ks;
}

// K slices the tiles of this size take for p (1: no split) and their depth.
template <typename T, int TM>
int64_t tile_slices(const GemmProblem &p, int64_t *kchunk) {
    constexpr int64_t BT = 32 * TM;
    const int64_t tm = (p.M + BT - 1) / BT, tn = (p.N + BT - 1) / BT;
    *kchunk = 0;
    return split_count<T, TM>(p, tm * tn * p.nb0 * p.nb1, kchunk);
}

// ext_part: the caller's [slices][z][m][n] buffer; the slices' raw sums go
// there (one slice when the product is not split) and no combine runs.
template <typename T, int TM>
int32_t run_tiles(const GemmProblem &p, int al, int bl, bool av, bool bv, hipStream_t st, T *ext_part = nullptr) {
    constexpr int64_t BT = 32 * TM;
    const int64_t tm = (p.M + BT - 1) / BT, tn = (p.N + BT - 1) / BT;
    const int64_t nz = p.nb0 * p.nb1;
    if (!grid_fits(tm * tn, THREADS) || nz > 65535) return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: grid too large");
    int64_t kchunk = 0;
    const int64_t ks = tile_slices<T, TM>(p, &kchunk);
    T *part = ext_part;
    const size_t part_bytes = ks > 1 && !ext_part ? (size_t)(ks * nz * p.M * p.N) * sizeof(T) : 0;
    if (ext_part) {
        // one slice spanning K when unsplit (a multiple of the tile depth)
        if (ks == 1) kchunk = (p.K + Depth<T, TM>::BK - 1) / Depth<T, TM>::BK * Depth<T, TM>::BK;
    } else if (ks > 1) {
        part = static_cast<T *>(scratch_alloc(part_bytes));
        if (!part) return set_error(CHELIS_HIP_EHIP, "matmul: split-K scratch of %zu bytes", part_bytes);
    } else {
        kchunk = 0;
    }
    const dim3 grid((unsigned)(tm * tn), (unsigned)nz, (unsigned)ks);
    switch (al * 3 + bl) {
        case 0: launch_mfma<T, 0, 0, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
        case 1: launch_mfma<T, 0, 1, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
        case 2: launch_mfma<T, 0, 2, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
        case 3: launch_mfma<T, 1, 0, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
        case 4: launch_mfma<T, 1, 1, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
        case 5: launch_mfma<T, 1, 2, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
        case 6: launch_mfma<T, 2, 0, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
        case 7: launch_mfma<T, 2, 1, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
        default: launch_mfma<T, 2, 2, TM>(p, grid, tm, tn, av, bv, part, kchunk, st); break;
    }
    if (ks > 1 && !ext_part) {
        int tpr = 1;
        while (tpr < 256 && 4 * tpr < p.N) tpr <<= 1;
        const int64_t rows = nz * p.M, blocks = (rows + 256 / tpr - 1) / (256 / tpr), cols = (p.N + 1023) / 1024;
        if (!grid_fits(blocks, 256) || cols > 65535) {
            scratch_free(part, part_bytes);
            return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: split-K combine grid too large");
        }
        if (combine_vec_ok<T>(p, nz))
            splitk_combine_kernel<T, true><<<dim3((unsigned)blocks, (unsigned)cols), 256, 0, st>>>(p, part, (int)ks,
                                                                                                   nz, tpr);
        else
            splitk_combine_kernel<T, false><<<dim3((unsigned)blocks, (unsigned)cols), 256, 0, st>>>(p, part, (int)ks,
                                                                                                    nz, tpr);
        scratch_free(part, part_bytes);
    }
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

// Tile size for p: 128-tiles (true) or 64-tiles.
template <typename T>
bool big_tiles(const GemmProblem &p) {
    // 128-tiles when they give every CU two tiles (the two workgroups a CU
    // holds), no dimension is at most half a tile and K runs long enough
    // (> 128) to amortize a tile's first loads and its epilogue; 64-tiles,
    // four times as many workgroups that overlap those phases, otherwise.
    // Measured: the transformer block's projections (256 128-tiles each,
    // K = 1024) take 87 us on 64-tiles against 94 us on 128-tiles; the 128 x
    // (512 x 512 x 64) attention scores 80 us against 132 us. With K of at
    // least 2048, 128-tiles split across K win instead: FFN2 (4096 x 1024 x
    // 4096, 256 128-tiles) takes 279 us as 2 slices of 128-tiles against
    // 305 us on 64-tiles.
    const int64_t cus = device_cus();
    const int64_t big = ((p.M + 127) / 128) * ((p.N + 127) / 128) * p.nb0 * p.nb1;
    const int64_t kslices = p.K / 1024 < 16 ? p.K / 1024 : 16;
    const bool few = big < 2 * cus && !(p.causal == 0 && p.K >= 2048 && big * kslices >= 2 * cus && big >= cus / 2);
    const bool small = few || p.M <= 64 || p.N <= 64 || p.K <= 128;
    return !small;
}

template <typename T>
int32_t run_mfma(const GemmProblem &p, hipStream_t st, T *ext_part = nullptr) {
    bool av = false, bv = false;
    const int al = lay_of<T>(p.sam, p.sak, p.a, p.M, p.K, &av);
    const int bl = lay_of<T>(p.sbn, p.sbk, p.b, p.N, p.K, &bv);
    return big_tiles<T>(p) ? run_tiles<T, 4>(p, al, bl, av, bv, st, ext_part)
                           : run_tiles<T, 2>(p, al, bl, av, bv, st, ext_part);
}

template <typename T>
int64_t mfma_slices(const GemmProblem &p) {
    int64_t kchunk = 0;
    return big_tiles<T>(p) ? tile_slices<T, 4>(p, &kchunk) : tile_slices<T, 2>(p, &kchunk);
}

}  // namespace

int32_t gemm_mfma(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    return dt == CHELIS_DTYPE_F32 ? run_mfma<float>(p, st) : run_mfma<double>(p, st);
}

int64_t gemm_mfma_slice_count(chelis_dtype dt, const GemmProblem &p) {
    return dt == CHELIS_DTYPE_F32 ? mfma_slices<float>(p) : mfma_slices<double>(p);
}

int32_t gemm_mfma_slices(chelis_dtype dt, const GemmProblem &p, void *part, hipStream_t st) {
    return dt == CHELIS_DTYPE_F32 ? run_mfma<float>(p, st, static_cast<float *>(part))
                                  : run_mfma<double>(p, st, static_cast<double *>(part));
}

}  // namespace chelis

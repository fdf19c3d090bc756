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

namespace chelis {
namespace {

constexpr int MAXD = 24;  // carry-stack depth: up to 2^24 segments

// Push one block total into a wave-uniform carry stack (count = index of
// this block). Unrolled with static indices so the stack stays in VGPRs.
template <typename T>
__device__ inline void carry_push(T (&lvl)[MAXD], int64_t count, T carry) {
    bool done = false;
#pragma unroll
    for (int d = 0; d < MAXD; ++d) {
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

template <typename T>
__device__ inline T carry_total(const T (&lvl)[MAXD], int64_t count) {
    T total = T(0);
    bool found = false;
#pragma unroll
    for (int d = 0; d < MAXD; ++d) {
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
// run is contiguous, aligned and complete.
template <typename T, int V, bool CONTIG>
__device__ inline void load_run(const T *__restrict__ p, int64_t s, int64_t k, int64_t K, bool vec_ok, T (&x)[V]) {
    if (CONTIG && vec_ok && k + V <= K) {
        constexpr int W = Vec16<T>::W;
#pragma unroll
        for (int q = 0; q < V / W; ++q) {
            typename Vec16<T>::type v = reinterpret_cast<const typename Vec16<T>::type *>(p)[q];
            const T *e = reinterpret_cast<const T *>(&v);
#pragma unroll
            for (int u = 0; u < W; ++u) x[q * W + u] = e[u];
        }
    } else {
#pragma unroll
        for (int u = 0; u < V; ++u) x[u] = (k + u < K) ? p[CONTIG ? u : u * s] : T(0);
    }
}

// ---------------------------------------------------------------- wave per output
// GEMV-class shapes: one wave streams one output's K products, 64*V leaves
// per segment, fully coalesced when the operand is K-contiguous.
template <typename T, int V, bool AK, bool BK>
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
    T lvl[MAXD];
    for (int64_t s = 0; s < nseg; ++s) {
        const int64_t k = s * SEG + (int64_t)lane * V;
        T a[V], b[V];
        load_run<T, V, AK>(A + k * p.sak, p.sak, k, p.K, a_vec, a);
        load_run<T, V, BK>(B + k * p.sbk, p.sbk, k, p.K, b_vec, b);
#pragma unroll
        for (int u = 0; u < V; ++u) a[u] = (k + u < p.K) ? a[u] * b[u] : T(-0.0);
        T x = tree_v<T, V>(a);
#pragma unroll
        for (int msk = 1; msk < 64; msk <<= 1) x = x + shfl_xor(x, msk);
        carry_push<T>(lvl, s, x);
    }
    if (lane == 0) {
        T *C = static_cast<T *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
        C[m * p.scm + n * p.scn] = gemm_epilogue<T>(carry_total<T>(lvl, nseg), p, z0, z1, m, n);
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
        carry_push<T>(lvl, s, x);
    }
    const int o = lane % P;
    if (lane < P) {
        const int64_t m = m_base + o / NJ, n = n0 + o % NJ;
        if (m < p.M && n < p.N) {
            T *C = static_cast<T *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
            C[m * p.scm + n * p.scn] = gemm_epilogue<T>(carry_total<T>(lvl, nseg), p, z0, z1, m, n);
        }
    }
}

// ---------------------------------------------------------------- thread per output
// Short K: one thread per output, leaves streamed straight into its carry
// stack (depth 12, K <= 4096), n fastest so B and C accesses coalesce.
constexpr int TD = 12;
template <typename T>
__global__ __launch_bounds__(256) void tree_thread_kernel(GemmProblem p, int64_t outputs) {
    const int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (w >= outputs) return;
    const int64_t n = w % p.N, mz = w / p.N, m = mz % p.M, z = mz / p.M;
    const int64_t z0 = z / p.nb1, z1 = z % p.nb1;
    const T *A = static_cast<const T *>(p.a) + z0 * p.sa0 + z1 * p.sa1 + m * p.sam;
    const T *B = static_cast<const T *>(p.b) + z0 * p.sb0 + z1 * p.sb1 + n * p.sbn;
    T lvl[TD];
    for (int64_t k = 0; k < p.K; ++k) {
        T carry = A[k * p.sak] * B[k * p.sbk];
        bool done = false;
#pragma unroll
        for (int d = 0; d < TD; ++d) {
            if (!done) {
                if ((k >> d) & 1) {
                    carry = lvl[d] + carry;
                } else {
                    lvl[d] = carry;
                    done = true;
                }
            }
        }
    }
    T total = T(0);
    bool found = false;
#pragma unroll
    for (int d = 0; d < TD; ++d)
        if ((p.K >> d) & 1) {
            total = found ? lvl[d] + total : lvl[d];
            found = true;
        }
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
    if (blocks > 0x7fffffffLL) return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: too many outputs");
    if (ak && bk) tree_wave_kernel<T, V, true, true><<<(unsigned)blocks, 256, 0, st>>>(p, outputs, av, bv);
    else if (ak) tree_wave_kernel<T, V, true, false><<<(unsigned)blocks, 256, 0, st>>>(p, outputs, av, bv);
    else if (bk) tree_wave_kernel<T, V, false, true><<<(unsigned)blocks, 256, 0, st>>>(p, outputs, av, bv);
    else tree_wave_kernel<T, V, false, false><<<(unsigned)blocks, 256, 0, st>>>(p, outputs, av, bv);
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
    if (gx > 0x7fffffffLL || gy > 65535 || gz > 65535) return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: grid too large");
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)gz);
    if (ak && kfast) tree_tiled_kernel<T, V, R, NJ, WAVES, true, true><<<grid, 64 * WAVES, 0, st>>>(p, av);
    else if (ak) tree_tiled_kernel<T, V, R, NJ, WAVES, true, false><<<grid, 64 * WAVES, 0, st>>>(p, av);
    else if (kfast) tree_tiled_kernel<T, V, R, NJ, WAVES, false, true><<<grid, 64 * WAVES, 0, st>>>(p, av);
    else tree_tiled_kernel<T, V, R, NJ, WAVES, false, false><<<grid, 64 * WAVES, 0, st>>>(p, av);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

template <typename T>
int32_t run_thread(const GemmProblem &p, hipStream_t st) {
    if (p.K > (int64_t(1) << TD)) return set_error(CHELIS_HIP_EDOMAIN, "matmul: short-K kernel holds K <= %d", 1 << TD);
    const int64_t outputs = p.M * p.N * p.nb0 * p.nb1;
    const int64_t blocks = (outputs + 255) / 256;
    if (blocks > 0x7fffffffLL) return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: too many outputs");
    tree_thread_kernel<T><<<(unsigned)blocks, 256, 0, st>>>(p, outputs);
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
int32_t gemm_tree_thread(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    return dt == CHELIS_DTYPE_F32 ? run_thread<float>(p, st) : run_thread<double>(p, st);
}

}  // namespace chelis

// bf16 / f16 matmul on the CDNA4 matrix cores, and the 16-bit <-> binary32
// conversions of the exact matmul path.
//
// spec/04 section 5.7.1 gives a 16-bit matmul a binary32 accumulator; the
// reference runs it on hipblasGemmEx with HIPBLAS_COMPUTE_32F and a 16-bit
// result (crates/chelis-backend-hip/runtime/chelis_hip_runtime.h:92-170).
// Here v_mfma_f32_16x16x32_bf16 / _f16 accumulate in binary32 and the
// epilogue encodes each result once (narrow.h: nearest even, canonical NaN).
//
// Tile: a 256-thread workgroup (4 waves, 2 x 2) owns 128 x 128 of C; each
// wave 64 x 64 = 4 x 4 blocks of 16 x 16. K moves in steps of 64 (two MFMA
// k-blocks of 32) through two LDS buffers holding both operands
// K-contiguous (As[m][k], Bs[n][k]) with a 144-byte row pitch, so the 8
// rows a 16-byte read phase touches fall on 8 disjoint 4-bank groups (one
// step of 64 measured 13-16 % faster than steps of 32 at 4096^3; a second
// register staging set pushed the registers to one wave per SIMD). An MFMA
// of shape 16x16x32 takes from lane q*16 + i
// the 8 values of row i (A) or column i (B) at k = 8q .. 8q + 7, one 16-byte
// LDS read, and pairs A and B entries of the same lane group and item, so
// both operands share one k map; it returns C[4q + r][j] in lane q*16 + j,
// item r (the 16x16 binary32 output layout of the 16x16x4 f32 MFMA, which
// the f32 kernel uses). The next step's global loads are in flight in
// registers while the matrix cores run the current one.
#include "gemm.h"
#include "narrow.h"

namespace chelis {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

template <Narrow K>
__device__ inline f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
    if constexpr (K == Narrow::Bf16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
}

constexpr int THREADS = 256, BM = 128, BN = 128, BK = 64, LD = 72;

// One operand tile [ROWS][BK] staged in registers: LAY 0 = vectors along K,
// 8 values per 16-byte vector, stored as they are; 2 = element by element.
// LAY 1 = vectors along the outer axis (M of A, N of B), which LDS wants
// K-contiguous: thread t owns the 4 x 8 block of outer rows 4 nb + e (e < 4)
// and k = 8 kb + u (u < 8), nb = t % 4 + 4 (t / 32), kb = (t / 4) % 8. It
// reads one 8-byte vector of 4 rows per k, transposes the block in
// registers (one byte permute per output word) and writes one 16-byte
// vector of 8 k per row: with the 144-byte row pitch, 16 consecutive lanes
// write 16 distinct 4-bank groups (rows 4 nb + e, columns 8 kb), where the
// former element-by-element 2-byte stores took 32 LDS writes per thread.
template <int LAY, int ROWS>
struct Stage16 {
    static constexpr int NV = ROWS * BK / 8 / THREADS;
    static_assert(LAY != 1 || ROWS * BK == 32 * THREADS, "one 4 x 8 block per thread");
    uint4 r[LAY == 1 ? 1 : NV];
    uint2 q[LAY == 1 ? 8 : 1];

    // element (row, k) at base[row * s_row + k * s_k]; CHECK = false: the
    // whole tile is inside the operand and the vectors are aligned.
    template <bool CHECK>
    __device__ void load(const uint16_t *__restrict__ base, int64_t s_row, int64_t s_k, int64_t row0, int64_t rows,
                         int64_t k0, int64_t K) {
        const int t = threadIdx.x;
        if constexpr (LAY == 1) {
            const int nb = t % 4 + 4 * (t / 32), kb = (t / 4) % 8;
            const int64_t gr = row0 + 4 * nb;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t gk = k0 + 8 * kb + u;
                const uint16_t *p = base + gr + gk * s_k;
                if (!CHECK || (gk < K && gr + 4 <= rows)) {
                    q[u] = *reinterpret_cast<const uint2 *>(p);
                } else {
                    uint16_t e[4];
#pragma unroll
                    for (int w = 0; w < 4; ++w) e[w] = (gk < K && gr + w < rows) ? p[w * s_row] : (uint16_t)0;
                    q[u] = __builtin_bit_cast(uint2, e);
                }
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int idx = t + THREADS * j;
            const int row = idx / (BK / 8), kv = (idx % (BK / 8)) * 8;
            const int64_t gr = row0 + row, gk = k0 + kv;
            const uint16_t *p = base + gr * s_row + gk * s_k;
            if (LAY == 0 && (!CHECK || (gr < rows && gk + 8 <= K))) {
                r[j] = *reinterpret_cast<const uint4 *>(p);
            } else {
                uint16_t e[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) e[u] = (gr < rows && gk + u < K) ? p[u * s_k] : (uint16_t)0;
                r[j] = __builtin_bit_cast(uint4, e);
            }
        }
    }

    __device__ void store(uint16_t *lds) const {
        const int t = threadIdx.x;
        if constexpr (LAY == 1) {
            const int nb = t % 4 + 4 * (t / 32), kb = (t / 4) % 8;
            // output row e, word w: k = 2w in the low half, 2w + 1 in the high
            uint32_t w[4][4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const uint32_t a0 = q[2 * h].x, a1 = q[2 * h].y, b0 = q[2 * h + 1].x, b1 = q[2 * h + 1].y;
                w[0][h] = (a0 & 0xffffu) | (b0 << 16);
                w[1][h] = (a0 >> 16) | (b0 & 0xffff0000u);
                w[2][h] = (a1 & 0xffffu) | (b1 << 16);
                w[3][h] = (a1 >> 16) | (b1 & 0xffff0000u);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                *reinterpret_cast<uint4 *>(lds + (4 * nb + e) * LD + 8 * kb) = uint4{w[e][0], w[e][1], w[e][2], w[e][3]};
            return;
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int idx = t + THREADS * j;
            const int row = idx / (BK / 8), kv = (idx % (BK / 8)) * 8;
            *reinterpret_cast<uint4 *>(lds + row * LD + kv) = r[j];
        }
    }
};

template <Narrow KIND, int ALAY, int BLAY>
__global__ __launch_bounds__(THREADS) void gemm16_kernel(GemmProblem p, int64_t tiles_m, int64_t tiles_n) {
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LD];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LD];

    // XCD-aware tile order: each XCD (workgroups are dealt round-robin) gets
    // one contiguous run of tiles, walked in groups of 8 tile-rows.
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

    const int64_t z = blockIdx.y;
    const int64_t z0 = z / p.nb1, z1 = z % p.nb1;
    const uint16_t *A = static_cast<const uint16_t *>(p.a) + z0 * p.sa0 + z1 * p.sa1;
    const uint16_t *B = static_cast<const uint16_t *>(p.b) + z0 * p.sb0 + z1 * p.sb1;
    const int64_t K = p.K;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, fq = lane >> 4;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{};

    Stage16<ALAY, BM> sa;
    Stage16<BLAY, BN> sb;
    const int64_t ksteps = (K + BK - 1) / BK;
    const bool inside = ALAY != 2 && BLAY != 2 && m0 + BM <= p.M && n0 + BN <= p.N && K >= BK && K % BK == 0;
    auto run = [&](auto check) {
        constexpr bool CK = decltype(check)::value;
        const int64_t last = ksteps - 1;
        sa.template load<CK>(A, p.sam, p.sak, m0, p.M, 0, K);
        sb.template load<CK>(B, p.sbn, p.sbk, n0, p.N, 0, K);
        sa.store(As[0]);
        sb.store(Bs[0]);
        __syncthreads();
        for (int64_t ks = 0; ks < ksteps; ++ks) {
            const int buf = (int)(ks & 1);
            // the next step's loads (the last step reloads itself: branch free)
            const int64_t kn = (ks < last ? ks + 1 : last) * BK;
            sa.template load<CK>(A, p.sam, p.sak, m0, p.M, kn, K);
            sb.template load<CK>(B, p.sbn, p.sbk, n0, p.N, kn, K);
#pragma unroll
            for (int kk = 0; kk < BK / 32; ++kk) {
                const uint16_t *as = As[buf] + (wm * 64 + fr) * LD + kk * 32 + fq * 8;
                const uint16_t *bs = Bs[buf] + (wn * 64 + fr) * LD + kk * 32 + fq * 8;
                uint4 af[4], bf[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const uint4 *>(as + i * 16 * LD);
#pragma unroll
                for (int j = 0; j < 4; ++j) bf[j] = *reinterpret_cast<const uint4 *>(bs + j * 16 * LD);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<KIND>(af[i], bf[j], acc[i][j]);
            }
            sa.store(As[buf ^ 1]);
            sb.store(Bs[buf ^ 1]);
            __syncthreads();
        }
    };
    if (inside) run(std::false_type{});
    else run(std::true_type{});

    uint16_t *C = static_cast<uint16_t *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * 64 + i * 16 + 4 * fq + r;
                const int64_t n = n0 + wn * 64 + j * 16 + fr;
                if (m < p.M && n < p.N) C[m * p.scm + n * p.scn] = f32_to_narrow<KIND>(acc[i][j][r]);
            }
}

// ---------------------------------------------------------------- deep
// The common interior case - A along K, B along K or along N, every tile
// whole, K a whole number of steps - in a kernel with two register staging
// sets: each step's global loads are issued two steps before their LDS store
// (one step in the kernel above), each step's fragments are read before its
// matrix work, and the registers are capped at two waves per SIMD. The
// staging registers are locals written and read in straight-line code (as
// arrays inside two staging objects the compiler kept them in scratch memory
// and waited for every load right after issuing it). The MFMA order is the
// kernel above's, so the bits are too. 4096^3 bf16 with both operands along
// K on one box: 161-196 against 146-170 us.
template <Narrow KIND, int BLAY>
__global__ __launch_bounds__(THREADS, 2) void gemm16_deep_kernel(GemmProblem p, int64_t tiles_m, int64_t tiles_n) {
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LD];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LD];
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
    const int64_t z = blockIdx.y;
    const int64_t z0 = z / p.nb1, z1 = z % p.nb1;
    const uint16_t *A = static_cast<const uint16_t *>(p.a) + z0 * p.sa0 + z1 * p.sa1;
    const uint16_t *B = static_cast<const uint16_t *>(p.b) + z0 * p.sb0 + z1 * p.sb1;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, fq = lane >> 4;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{};

    // A (and B along K): thread t stages rows t / 8 + 32 j (j < 4), k = 8 (t % 8) ..
    // B along N: the 4 x 8 block of rows 4 nb .. and k = 8 kb .. (the LAY 1 map above)
    const int srow = t >> 3, skv = (t & 7) * 8;
    const int nb = t % 4 + 4 * (t / 32), kb = (t / 4) % 8;
    const uint16_t *ga = A + (m0 + srow) * p.sam + skv;
    const uint16_t *gb = BLAY == 0 ? B + (n0 + srow) * p.sbn + skv : B + n0 + 4 * nb + (int64_t)(8 * kb) * p.sbk;
    const int64_t ra = 32 * p.sam, rb = BLAY == 0 ? 32 * p.sbn : p.sbk;
    const int64_t bstep = BLAY == 0 ? BK : BK * p.sbk;  // B elements from one step to the next
    const int aoff = srow * LD + skv, boff = BLAY == 0 ? srow * LD + skv : 4 * nb * LD + 8 * kb;
    const int64_t ksteps = p.K / BK, last = ksteps - 1;

    uint4 xa0, xa1, xa2, xa3, ya0, ya1, ya2, ya3;  // A, sets x and y
    uint4 xb0, xb1, xb2, xb3, yb0, yb1, yb2, yb3;  // B along K
    uint2 xq[8], yq[8];                            // B along N
#define CHELIS_D_LOADA(S, V0, V1, V2, V3)                                                  \
    do {                                                                                   \
        const uint16_t *g_ = ga + ((S) < last ? (S) : last) * BK;                          \
        V0 = *reinterpret_cast<const uint4 *>(g_);                                         \
        V1 = *reinterpret_cast<const uint4 *>(g_ + ra);                                    \
        V2 = *reinterpret_cast<const uint4 *>(g_ + 2 * ra);                                \
        V3 = *reinterpret_cast<const uint4 *>(g_ + 3 * ra);                                \
    } while (0)
#define CHELIS_D_STORE4(L, V0, V1, V2, V3)                                                 \
    do {                                                                                   \
        *reinterpret_cast<uint4 *>(L) = V0;                                                \
        *reinterpret_cast<uint4 *>((L) + 32 * LD) = V1;                                    \
        *reinterpret_cast<uint4 *>((L) + 64 * LD) = V2;                                    \
        *reinterpret_cast<uint4 *>((L) + 96 * LD) = V3;                                    \
    } while (0)
#define CHELIS_D_LOADB(S, V0, V1, V2, V3, Q)                                               \
    do {                                                                                   \
        const uint16_t *g_ = gb + ((S) < last ? (S) : last) * bstep;                       \
        if constexpr (BLAY == 0) {                                                         \
            V0 = *reinterpret_cast<const uint4 *>(g_);                                     \
            V1 = *reinterpret_cast<const uint4 *>(g_ + rb);                                \
            V2 = *reinterpret_cast<const uint4 *>(g_ + 2 * rb);                            \
            V3 = *reinterpret_cast<const uint4 *>(g_ + 3 * rb);                            \
        } else {                                                                           \
            _Pragma("unroll") for (int u_ = 0; u_ < 8; ++u_)                               \
                Q[u_] = *reinterpret_cast<const uint2 *>(g_ + u_ * rb);                    \
        }                                                                                  \
    } while (0)
#define CHELIS_D_STOREB(L, V0, V1, V2, V3, Q)                                              \
    do {                                                                                   \
        if constexpr (BLAY == 0) {                                                         \
            CHELIS_D_STORE4(L, V0, V1, V2, V3);                                            \
        } else {                                                                           \
            _Pragma("unroll") for (int e_ = 0; e_ < 4; ++e_) {                             \
                uint32_t w_[4];                                                            \
                _Pragma("unroll") for (int h_ = 0; h_ < 4; ++h_) {                         \
                    const uint32_t lo_ = e_ & 1 ? Q[2 * h_].x >> 16 : Q[2 * h_].x & 0xffffu;       \
                    const uint32_t lo2_ = e_ & 1 ? Q[2 * h_].y >> 16 : Q[2 * h_].y & 0xffffu;      \
                    const uint32_t hi_ = e_ & 1 ? Q[2 * h_ + 1].x & 0xffff0000u : Q[2 * h_ + 1].x << 16; \
                    const uint32_t hi2_ = e_ & 1 ? Q[2 * h_ + 1].y & 0xffff0000u : Q[2 * h_ + 1].y << 16; \
                    w_[h_] = e_ < 2 ? (lo_ | hi_) : (lo2_ | hi2_);                         \
                }                                                                          \
                *reinterpret_cast<uint4 *>((L) + e_ * LD) = uint4{w_[0], w_[1], w_[2], w_[3]};  \
            }                                                                              \
        }                                                                                  \
    } while (0)
    // one step: step KS's matrix work from buffer KS % 2, then the set holding
    // step KS + 1 goes to the other buffer and refills with step KS + 3
#define CHELIS_D_STEP(KS, A0, A1, A2, A3, B0, B1, B2, B3, Q)                               \
    do {                                                                                   \
        const int buf_ = (int)((KS) & 1);                                                  \
        uint4 af_[2][4], bf_[2][4];                                                        \
        _Pragma("unroll") for (int kk_ = 0; kk_ < 2; ++kk_) {                              \
            const uint16_t *as_ = As[buf_] + (wm * 64 + fr) * LD + kk_ * 32 + fq * 8;      \
            const uint16_t *bs_ = Bs[buf_] + (wn * 64 + fr) * LD + kk_ * 32 + fq * 8;      \
            _Pragma("unroll") for (int i_ = 0; i_ < 4; ++i_)                               \
                af_[kk_][i_] = *reinterpret_cast<const uint4 *>(as_ + i_ * 16 * LD);       \
            _Pragma("unroll") for (int j_ = 0; j_ < 4; ++j_)                               \
                bf_[kk_][j_] = *reinterpret_cast<const uint4 *>(bs_ + j_ * 16 * LD);       \
        }                                                                                  \
        _Pragma("unroll") for (int kk_ = 0; kk_ < 2; ++kk_)                                \
            _Pragma("unroll") for (int i_ = 0; i_ < 4; ++i_)                               \
                _Pragma("unroll") for (int j_ = 0; j_ < 4; ++j_)                           \
                    acc[i_][j_] = mfma16<KIND>(af_[kk_][i_], bf_[kk_][j_], acc[i_][j_]);   \
        CHELIS_D_STORE4(As[buf_ ^ 1] + aoff, A0, A1, A2, A3);                              \
        CHELIS_D_STOREB(Bs[buf_ ^ 1] + boff, B0, B1, B2, B3, Q);                           \
        __syncthreads();                                                                   \
        CHELIS_D_LOADA((KS) + 3, A0, A1, A2, A3);                                          \
        CHELIS_D_LOADB((KS) + 3, B0, B1, B2, B3, Q);                                       \
    } while (0)

    // steps 0 (stored), 1 (set y) and 2 (set x) in flight before the loop
    CHELIS_D_LOADA(0, xa0, xa1, xa2, xa3);
    CHELIS_D_LOADB(0, xb0, xb1, xb2, xb3, xq);
    CHELIS_D_STORE4(As[0] + aoff, xa0, xa1, xa2, xa3);
    CHELIS_D_STOREB(Bs[0] + boff, xb0, xb1, xb2, xb3, xq);
    CHELIS_D_LOADA(1, ya0, ya1, ya2, ya3);
    CHELIS_D_LOADB(1, yb0, yb1, yb2, yb3, yq);
    CHELIS_D_LOADA(2, xa0, xa1, xa2, xa3);
    CHELIS_D_LOADB(2, xb0, xb1, xb2, xb3, xq);
    __syncthreads();
    int64_t ks = 0;
    for (; ks + 1 < ksteps; ks += 2) {
        CHELIS_D_STEP(ks, ya0, ya1, ya2, ya3, yb0, yb1, yb2, yb3, yq);
        CHELIS_D_STEP(ks + 1, xa0, xa1, xa2, xa3, xb0, xb1, xb2, xb3, xq);
    }
    if (ks < ksteps) CHELIS_D_STEP(ks, ya0, ya1, ya2, ya3, yb0, yb1, yb2, yb3, yq);
#undef CHELIS_D_STEP
#undef CHELIS_D_STOREB
#undef CHELIS_D_LOADB
#undef CHELIS_D_STORE4
#undef CHELIS_D_LOADA

    uint16_t *C = static_cast<uint16_t *>(p.c) + z0 * p.sc0 + z1 * p.sc1;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * 64 + i * 16 + 4 * fq + r;
                const int64_t n = n0 + wn * 64 + j * 16 + fr;
                C[m * p.scm + n * p.scn] = f32_to_narrow<KIND>(acc[i][j][r]);
            }
}

// Staging layout of an operand: vectors along K (0) or along its outer
// axis (1) when that axis has unit stride, the other stride and every batch
// offset keep 16-byte alignment, and the base is aligned; else 2.
int lay_of(const void *base, int64_t s_outer, int64_t s_k, int64_t s0, int64_t s1) {
    const bool aligned = (reinterpret_cast<uintptr_t>(base) & 15u) == 0 && s0 % 8 == 0 && s1 % 8 == 0;
    if (aligned && s_k == 1 && s_outer % 8 == 0) return 0;
    if (aligned && s_outer == 1 && s_k % 8 == 0) return 1;
    return 2;
}

template <Narrow KIND, int ALAY, int BLAY>
void launch16(const GemmProblem &p, dim3 grid, int64_t tm, int64_t tn, hipStream_t st) {
    gemm16_kernel<KIND, ALAY, BLAY><<<grid, THREADS, 0, st>>>(p, tm, tn);
}

template <Narrow KIND>
int32_t gemm16_kind(const GemmProblem &p, hipStream_t st) {
    const int64_t tm = (p.M + BM - 1) / BM, tn = (p.N + BN - 1) / BN;
    const int64_t nz = p.nb0 * p.nb1;
    if (!grid_fits(tm * tn, 256) || nz > 65535) return set_error(CHELIS_HIP_EUNSUPPORTED, "matmul: grid too large");
    const dim3 grid((unsigned)(tm * tn), (unsigned)nz);
    const int la = lay_of(p.a, p.sam, p.sak, p.sa0, p.sa1), lb = lay_of(p.b, p.sbn, p.sbk, p.sb0, p.sb1);
    // whole tiles and whole steps with A along K: the deep kernel
    const bool whole = p.M % BM == 0 && p.N % BN == 0 && p.K % BK == 0 && p.K > 0;
    if (whole && la == 0 && lb == 0) {
        gemm16_deep_kernel<KIND, 0><<<grid, THREADS, 0, st>>>(p, tm, tn);
        CHELIS_LAUNCH_CHECK();
        return CHELIS_HIP_OK;
    }
    if (whole && la == 0 && lb == 1) {
        gemm16_deep_kernel<KIND, 1><<<grid, THREADS, 0, st>>>(p, tm, tn);
        CHELIS_LAUNCH_CHECK();
        return CHELIS_HIP_OK;
    }
    // instantiated layouts: both K-contiguous, A K-contiguous with B along N
    // (row-major operands), and the element-by-element fallback
    if (la == 0 && lb == 0) launch16<KIND, 0, 0>(p, grid, tm, tn, st);
    else if (la == 0 && lb == 1) launch16<KIND, 0, 1>(p, grid, tm, tn, st);
    else if (la == 1 && lb == 0) launch16<KIND, 1, 0>(p, grid, tm, tn, st);
    else if (la == 1 && lb == 1) launch16<KIND, 1, 1>(p, grid, tm, tn, st);
    else launch16<KIND, 2, 2>(p, grid, tm, tn, st);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

// The kernels below that index by thread run 256 threads per workgroup
// (their launches pass that count): the constant, not blockDim.x, which
// is a vector load from the dispatch packet at the start of each wave.
constexpr int kConvThreads = 256;

// dst[z][r][c] = src[z0 * s0 + z1 * s1 + r * sr + c * sc] widened to binary32
// (z = z0 * nz1 + z1; dst contiguous).
template <Narrow KIND>
__global__ __launch_bounds__(256) void widen_kernel(const uint16_t *__restrict__ src, float *__restrict__ dst,
                                                    int64_t nz1, int64_t rows, int64_t cols, int64_t s0, int64_t s1,
                                                    int64_t sr, int64_t sc, int64_t count) {
    const int64_t stride = (int64_t)gridDim.x * kConvThreads;
    for (int64_t i = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < count; i += stride) {
        const int64_t c = i % cols, r = (i / cols) % rows, z = i / (cols * rows);
        dst[i] = narrow_to_f32<KIND>(src[(z / nz1) * s0 + (z % nz1) * s1 + r * sr + c * sc]);
    }
}

// dst[z0 * s0 + z1 * s1 + r * sr + c * sc] = src[z][r][c] encoded to 16 bits.
template <Narrow KIND>
__global__ __launch_bounds__(256) void narrow_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                     int64_t nz1, int64_t rows, int64_t cols, int64_t s0, int64_t s1,
                                                     int64_t sr, int64_t sc, int64_t count) {
    const int64_t stride = (int64_t)gridDim.x * kConvThreads;
    for (int64_t i = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; i < count; i += stride) {
        const int64_t c = i % cols, r = (i / cols) % rows, z = i / (cols * rows);
        dst[(z / nz1) * s0 + (z % nz1) * s1 + r * sr + c * sc] = f32_to_narrow<KIND>(src[i]);
    }
}

unsigned blocks_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    return (unsigned)(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

}  // namespace

int32_t gemm_mfma16(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    return dt == CHELIS_DTYPE_BF16 ? gemm16_kind<Narrow::Bf16>(p, st) : gemm16_kind<Narrow::F16>(p, st);
}

int32_t widen16(chelis_dtype dt, const void *src, float *dst, int64_t nz0, int64_t nz1, int64_t rows, int64_t cols,
                int64_t s0, int64_t s1, int64_t sr, int64_t sc, hipStream_t st) {
    const int64_t n = nz0 * nz1 * rows * cols;
    if (!n) return CHELIS_HIP_OK;
    if (dt == CHELIS_DTYPE_BF16)
        widen_kernel<Narrow::Bf16><<<blocks_for(n), 256, 0, st>>>((const uint16_t *)src, dst, nz1, rows, cols, s0, s1,
                                                                  sr, sc, n);
    else
        widen_kernel<Narrow::F16><<<blocks_for(n), 256, 0, st>>>((const uint16_t *)src, dst, nz1, rows, cols, s0, s1,
                                                                 sr, sc, n);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

int32_t narrow16(chelis_dtype dt, const float *src, void *dst, int64_t nz0, int64_t nz1, int64_t rows, int64_t cols,
                 int64_t s0, int64_t s1, int64_t sr, int64_t sc, hipStream_t st) {
    const int64_t n = nz0 * nz1 * rows * cols;
    if (!n) return CHELIS_HIP_OK;
    if (dt == CHELIS_DTYPE_BF16)
        narrow_kernel<Narrow::Bf16><<<blocks_for(n), 256, 0, st>>>(src, (uint16_t *)dst, nz1, rows, cols, s0, s1, sr,
                                                                   sc, n);
    else
        narrow_kernel<Narrow::F16><<<blocks_for(n), 256, 0, st>>>(src, (uint16_t *)dst, nz1, rows, cols, s0, s1, sr,
                                                                  sc, n);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

}  // namespace chelis

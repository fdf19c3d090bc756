// The linear-regression gradient step (config 1) in two launches instead of
// eight:
//   r = X.w - y;  grad = (X^T.r) / n;  loss = tree(r * r) / n
// with every value rounded as the unfused graph rounds it, so the results
// are bit-identical to the matmul / chain / reduction launches they replace
// (and to the C lane):
//   * X.w is a contraction of d <= 32 terms: the products, padded with -0.0
//     to a power of two, summed as one register tree, the total finalized;
//   * r = canon(Xw - y);
//   * X^T.r and tree(r * r) are sums over the n rows in the canonical
//     adjacent-pair tree. The first launch sums aligned blocks of 64 rows
//     (the aligned subtrees of the canonical tree; rows past n are -0.0
//     leaves, which leave the carry tree's values unchanged), the second
//     joins the block totals pairwise in LDS and divides by n.
#include "gemm.h"

namespace chelis {
namespace {

constexpr int kMaxD = 32;
constexpr int kRowsPerBlock = 64;      // one wave per block of rows (2^6: six tree levels)
constexpr int kMaxBlocks = 4096;       // block totals the joining pass holds in LDS

// part[j][block], j < d: the block's sum of X[i][j] * r_i; part[d][block]:
// its sum of canon(r_i * r_i). Each lane owns one row; the leaves go to LDS
// and are joined there level by level, adjacent pairs first (the aligned
// 64-leaf subtree of the canonical tree).
template <typename T, int P, bool VEC>
__global__ __launch_bounds__(kRowsPerBlock) void linreg_blocks_kernel(const T *__restrict__ X, int64_t ldx,
                                                                      const T *__restrict__ w, int64_t sw,
                                                                      const T *__restrict__ y, int64_t sy, int64_t n,
                                                                      int d, int64_t blocks, T *__restrict__ part) {
    __shared__ T leaves[kMaxD + 1][kRowsPerBlock + 1];
    const int lane = threadIdx.x;
    const int64_t i = (int64_t)blockIdx.x * kRowsPerBlock + lane;
    const bool in = i < n;
    const T *row = X + (in ? i : 0) * ldx;
    T x[P];
    if constexpr (VEC && P >= 2) {
        // rows are 16-byte aligned and d == P: P / V vector loads
        constexpr int V = 16 / (int)sizeof(T);
#pragma unroll
        for (int k = 0; k < P; k += V) {
            if constexpr (sizeof(T) == 8) {
                const double2 v = *reinterpret_cast<const double2 *>(row + k);
                x[k] = v.x;
                x[k + 1] = v.y;
            } else {
                const float4 v = *reinterpret_cast<const float4 *>(row + k);
                x[k] = v.x;
                x[k + 1] = v.y;
                x[k + 2] = v.z;
                x[k + 3] = v.w;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < P; ++k) x[k] = k < d ? row[k] : T(0);
    }
    // X.w: the products, -0.0 past d, one register tree
    T a[P];
#pragma unroll
    for (int k = 0; k < P; ++k) a[k] = k < d ? x[k] * w[k * sw] : T(-0.0);
#pragma unroll
    for (int s = 1; s < P; s <<= 1)
#pragma unroll
        for (int k = 0; k + s < P; k += 2 * s) a[k] = a[k] + a[k + s];
    const T xw = canon(d == 0 ? T(0) : a[0]);
    const T r = in ? canon(xw - y[i * sy]) : T(0);
#pragma unroll
    for (int j = 0; j < P; ++j)
        if (j < d) leaves[j][lane] = in ? x[j] * r : T(-0.0);
    leaves[d][lane] = in ? canon(r * r) : T(-0.0);
    __syncthreads();
    // level by level over the d + 1 columns: pair (2p, 2p + 1) of the level
#pragma unroll
    for (int ls = 0; ls < 6; ++ls) {
        const int s = 1 << ls, lp = 5 - ls;  // 2^lp pairs per column at this level
        for (int e = lane; e < ((d + 1) << lp); e += kRowsPerBlock) {
            const int j = e >> lp, q = (e & ((1 << lp) - 1)) << (ls + 1);
            leaves[j][q] = leaves[j][q] + leaves[j][q + s];
        }
        __syncthreads();
    }
    if (lane <= d) part[(int64_t)lane * blocks + blockIdx.x] = leaves[lane][0];
}

// One workgroup per value: its block totals (padded with -0.0 to a power
// of two, which keeps the carry tree's value) joined pairwise in LDS,
// finalized, then divided by n.
template <typename T>
__global__ __launch_bounds__(256) void linreg_finish_kernel(const T *__restrict__ part, int64_t blocks, int64_t pow2,
                                                            int d, T extent, T *__restrict__ grad, int64_t sg,
                                                            T *__restrict__ loss) {
    __shared__ T t[kMaxBlocks];
    const int j = blockIdx.x;
    for (int64_t b = threadIdx.x; b < pow2; b += 256) t[b] = b < blocks ? part[(int64_t)j * blocks + b] : T(-0.0);
    __syncthreads();
    for (int64_t s = 1; s < pow2; s <<= 1) {
        for (int64_t q = threadIdx.x * 2 * s; q < pow2; q += 256 * 2 * s) t[q] = t[q] + t[q + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const T q = canon(canon(t[0]) / extent);
        if (j < d) grad[j * sg] = q;
        else *loss = q;
    }
}

template <typename T, int P>
void launch_blocks(bool vec, unsigned g, const T *Xp, int64_t ldx, const T *wp, int64_t sw, const T *yp, int64_t sy,
                   int64_t n, int d, int64_t blocks, T *part, hipStream_t st) {
    if (vec) linreg_blocks_kernel<T, P, true><<<g, kRowsPerBlock, 0, st>>>(Xp, ldx, wp, sw, yp, sy, n, d, blocks, part);
    else linreg_blocks_kernel<T, P, false><<<g, kRowsPerBlock, 0, st>>>(Xp, ldx, wp, sw, yp, sy, n, d, blocks, part);
}

template <typename T>
int32_t run_linreg(const chelis_gpu_tensor *X, const chelis_gpu_tensor *w, const chelis_gpu_tensor *y,
                   const chelis_gpu_tensor *grad, const chelis_gpu_tensor *loss, hipStream_t st) {
    const int64_t n = X->shape[0];
    const int d = (int)X->shape[1];
    const int64_t blocks = (n + kRowsPerBlock - 1) / kRowsPerBlock;
    int64_t pow2 = 1;
    while (pow2 < blocks) pow2 <<= 1;
    const size_t part_bytes = (size_t)blocks * (d + 1) * sizeof(T);
    T *part = static_cast<T *>(scratch_alloc(part_bytes));
    if (!part) return set_error(CHELIS_HIP_EHIP, "linreg_step: scratch of %zu bytes", part_bytes);
    const T *Xp = static_cast<const T *>(X->data);
    const T *wp = static_cast<const T *>(w->data);
    const T *yp = static_cast<const T *>(y->data);
    const int64_t ldx = X->strides[0], sw = w->strides[0], sy = y->strides[0];
    const int64_t V = 16 / (int64_t)sizeof(T);
    const bool pow2d = (d & (d - 1)) == 0 && d >= V;
    const bool vec = pow2d && (reinterpret_cast<uintptr_t>(Xp) % 16) == 0 && ldx % V == 0;
    const unsigned g = (unsigned)blocks;
    if (d <= 1) launch_blocks<T, 1>(false, g, Xp, ldx, wp, sw, yp, sy, n, d, blocks, part, st);
    else if (d <= 2) launch_blocks<T, 2>(vec, g, Xp, ldx, wp, sw, yp, sy, n, d, blocks, part, st);
    else if (d <= 4) launch_blocks<T, 4>(vec, g, Xp, ldx, wp, sw, yp, sy, n, d, blocks, part, st);
    else if (d <= 8) launch_blocks<T, 8>(vec, g, Xp, ldx, wp, sw, yp, sy, n, d, blocks, part, st);
    else if (d <= 16) launch_blocks<T, 16>(vec, g, Xp, ldx, wp, sw, yp, sy, n, d, blocks, part, st);
    else launch_blocks<T, 32>(vec, g, Xp, ldx, wp, sw, yp, sy, n, d, blocks, part, st);
    linreg_finish_kernel<T><<<(unsigned)(d + 1), 256, 0, st>>>(part, blocks, pow2, d, (T)n,
                                                                 static_cast<T *>(grad->data), grad->strides[0],
                                                                 static_cast<T *>(loss->data));
    scratch_free(part, part_bytes);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

}  // namespace

bool linreg_fused_fits(const chelis_gpu_tensor *X, const chelis_gpu_tensor *w) {
    // d <= 32 (the short-K contraction); at most kMaxBlocks row blocks
    // (262 144 rows), the totals the joining pass keeps in LDS
    return X->rank == 2 && X->shape[1] >= 1 && X->shape[1] <= kMaxD && X->shape[0] >= 1 &&
           X->shape[0] <= (int64_t)kMaxBlocks * kRowsPerBlock && X->strides[1] == 1 && w->rank == 1;
}

int32_t linreg_fused(const chelis_gpu_tensor *X, const chelis_gpu_tensor *w, const chelis_gpu_tensor *y,
                     const chelis_gpu_tensor *grad, const chelis_gpu_tensor *loss, hipStream_t st) {
    return X->dtype == CHELIS_DTYPE_F32 ? run_linreg<float>(X, w, y, grad, loss, st)
                                        : run_linreg<double>(X, w, y, grad, loss, st);
}

}  // namespace chelis

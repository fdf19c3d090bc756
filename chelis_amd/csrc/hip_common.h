// Internal helpers shared by the gfx950 kernel families and their launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "chelis_hip.h"
#include "devmath.h"

namespace chelis {

// ---- host side ---------------------------------------------------------
int32_t set_error(int32_t status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
hipStream_t stream();
// Compute units of the current device (cached per device; 256 on MI355X).
int device_cus();

#define CHELIS_HIP_TRY(expr)                                                              \
    do {                                                                                  \
        hipError_t chelis_e_ = (expr);                                                    \
        if (chelis_e_ != hipSuccess)                                                      \
            return ::chelis::set_error(CHELIS_HIP_EHIP, "%s: %s", #expr,                  \
                                       hipGetErrorString(chelis_e_));                     \
    } while (0)

#define CHELIS_LAUNCH_CHECK()                                                             \
    do {                                                                                  \
        hipError_t chelis_e_ = hipGetLastError();                                         \
        if (chelis_e_ != hipSuccess)                                                      \
            return ::chelis::set_error(CHELIS_HIP_EHIP, "kernel launch: %s",              \
                                       hipGetErrorString(chelis_e_));                     \
    } while (0)

inline bool is_float(chelis_dtype d) { return d == CHELIS_DTYPE_F32 || d == CHELIS_DTYPE_F64; }
inline int64_t dtype_width(chelis_dtype d) {
    switch (d) {
        case CHELIS_DTYPE_F32: case CHELIS_DTYPE_I32: return 4;
        case CHELIS_DTYPE_F64: case CHELIS_DTYPE_I64: case CHELIS_DTYPE_KEY: return 8;
        case CHELIS_DTYPE_BOOL: case CHELIS_DTYPE_I8: return 1;
        case CHELIS_DTYPE_BF16: case CHELIS_DTYPE_F16: case CHELIS_DTYPE_I16: return 2;
        default: return 0;
    }
}

// Validate a packet: non-null, sane rank/shape/strides, count consistent,
// every reachable element inside byte_capacity.
int32_t check_tensor(const chelis_gpu_tensor *t, const char *name);
bool is_contiguous(const chelis_gpu_tensor *t);
bool same_shape(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b);

// A [rows, n] view of a tensor whose last axis is contiguous (stride 1) and
// whose leading axes collapse to one row index with a uniform row stride.
struct RowView {
    int64_t rows = 0, n = 0, ld = 0;
};
bool row_view(const chelis_gpu_tensor *t, RowView *v);

// dst (contiguous, count elements of `width` bytes) = src viewed through
// shape/strides; enqueued on `st`.
int32_t gather_contiguous(const void *src, void *dst, int32_t rank, const int64_t *shape, const int64_t *strides,
                          int64_t width, int64_t count, hipStream_t st);

inline unsigned grid_for(int64_t work, int per_block) {
    int64_t g = (work + per_block - 1) / per_block;
    return (unsigned)(g < 1 ? 1 : g);
}

// ---- device side -------------------------------------------------------
// Wave64 butterfly exchange.
template <typename T>
__device__ inline T shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// [05-OP-12] combine of two adjacent partial maxima, `a` covering the
// earlier indices: the first NaN wins with its bits, then the larger value,
// and on equality the earlier stored representation.
template <typename T>
__device__ inline T max_first(T a, T b) {
    if (a != a) return a;
    if (b != b) return b;
    return b > a ? b : a;
}
template <typename T>
__device__ inline T min_first(T a, T b) {
    if (a != a) return a;
    if (b != b) return b;
    return b < a ? b : a;
}

}  // namespace chelis

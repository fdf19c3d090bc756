// Internal helpers shared by the gfx950 kernel families and their launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "chelis_hip.h"
#include "devmath.h"
#include "launch_limits.h"

namespace chelis {

// ---- host side ---------------------------------------------------------
int32_t set_error(int32_t status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
hipStream_t stream();
// The library-wide exact mode (chelis_hip_set_exact): when set, every
// launcher that has the C lane's primitive for its result uses it (matmuls
// on the canonical-tree kernels, binary64 softmax rows with the correctly
// rounded exp and the IEEE division), so results are bit-identical to the
// C lane's; when clear, the default MFMA products and faithful binary64
// softmax rows, within the stated tolerances.
bool exact_mode();
// Pins the numeric mode for the calling thread's enqueues while it lives,
// so one entry (a program, a DAG run, a matmul dispatch) reads one mode
// throughout even if another thread switches the library-wide mode
// meanwhile. mode 0 / 1: that mode; -1: the mode an enclosing scope
// pinned, else the library-wide mode read once now.
class ModeScope {
  public:
    explicit ModeScope(int32_t mode = -1);
    ~ModeScope();
    ModeScope(const ModeScope &) = delete;
    ModeScope &operator=(const ModeScope &) = delete;

  private:
    int32_t prev_;
};
// Compute units of the current device (cached per device; 256 on MI355X).
int device_cus();
// The current device's two status words (device memory; *host, when given,
// receives a pinned host word for reading one back): [0] synchronous error
// codes, [1] the deferred trap channel. Null when the device has none.
int32_t *status_words(int32_t **host);
// Scratch device memory for work enqueued on the current device's library
// stream: blocks are recycled in stream order (a freed block's earlier users
// are already enqueued ahead of any later user) and cached for reuse, so
// the hot path makes no allocation calls. scratch_free takes the size given
// to scratch_alloc. Returns null when the device cannot allocate.
void *scratch_alloc(size_t bytes);
// hipMalloc, counted (chelis_hip_allocation_counts): every device allocation
// the library makes goes through it.
hipError_t device_malloc(void **p, size_t bytes);
void scratch_free(void *p, size_t bytes);
// Storage of owned device tensors (chelis_device_tensor_alloc): cached
// blocks for sizes up to 256 MiB; the free waits for the device first.
void *owner_block_alloc(size_t bytes);
hipError_t owner_block_free(void *p, size_t bytes);

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
// bfloat16 / binary16: 16-bit storage computed at binary32 (narrow.h).
inline bool is_narrow16(chelis_dtype d) { return d == CHELIS_DTYPE_BF16 || d == CHELIS_DTYPE_F16; }
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

// Keyed dropout (and, applied to a cotangent, its replay) with the key read
// on the device from key_dev, the storage of a KEY tensor: no host round trip.
// [05-OP-37]'s drop test unit < rate at the dtype, as an integer cut-off:
// an element is dropped exactly when its word >> 11 is below the result.
uint64_t dropout_cut(double rate, chelis_dtype dt);
// uniform_like with the key given on the host (key_dev null) or read on the
// device from key_dev.
int32_t uniform_like_run(uint64_t key, const uint64_t *key_dev, double low, double high,
                         const chelis_gpu_tensor *out);
int32_t dropout_device_key(const uint64_t *key_dev, const chelis_gpu_tensor *x, double rate,
                           const chelis_gpu_tensor *y);

// One FusedElem chain over n_groups independent (inputs, output) groups in
// as few launches as possible: inputs holds n_groups runs of n_inputs
// packets. Groups whose operands all stream with their output (or are one
// broadcast element) share a launch, four at a time; any other group runs
// through chelis_hip_fused_elementwise. Same bits as one call per group.
int32_t fused_elementwise_groups(const chelis_fused_chain *chain, int32_t n_inputs,
                                 const chelis_gpu_tensor *const *inputs, const chelis_gpu_tensor *const *outs,
                                 int32_t n_groups);

// grid_for / grid_fits: launch_limits.h

// ---- device side -------------------------------------------------------
// Wave64 butterfly exchange.
template <typename T>
__device__ inline T shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// ---- wave64 joins through DPP (VALU only, no LDS traffic) ----------------
// Every lane of the wave must be active. A butterfly join of aligned lane
// blocks: after level m every lane of an aligned 2^m-lane block holds the
// same block value, so ANY lane of the sibling block is a valid partner.
// Levels 1 and 2 use quad permutes (xor 1, xor 2), levels 3 and 4 the half
// mirror (lane i <-> 7 - i in each 8) and mirror (i <-> 15 - i in each 16)
// of a 16-lane DPP row, and the four row values are read into scalars and
// joined as (r0 + r1) + (r2 + r3). For a sum this is exactly the canonical
// adjacent-pair tree over the 64 lanes in lane order.
enum : int { kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140 };

template <int CTRL>
__device__ inline float dpp_perm(float v) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ inline double dpp_perm(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ inline float read_lane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ inline double read_lane(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Canonical tree sum of one value per lane (lane order = leaf order); every
// lane gets the total. IEEE addition is commutative, so both partners of a
// join compute the same bits.
template <typename T>
__device__ inline T wave_tree_sum(T x) {
    x = x + dpp_perm<kDppXor1>(x);
    x = x + dpp_perm<kDppXor2>(x);
    x = x + dpp_perm<kDppHalfMirror>(x);
    x = x + dpp_perm<kDppMirror>(x);
    return (read_lane(x, 0) + read_lane(x, 16)) + (read_lane(x, 32) + read_lane(x, 48));
}

// Plain IEEE maximum (v_max: a NaN operand yields the other one) over the
// wave; every lane gets it.
template <typename T>
__device__ inline T vmax(T a, T b) {
    if constexpr (sizeof(T) == 4) return __builtin_fmaxf(a, b);
    else return __builtin_fmax(a, b);
}
template <typename T>
__device__ inline T wave_vmax(T x) {
    x = vmax(x, dpp_perm<kDppXor1>(x));
    x = vmax(x, dpp_perm<kDppXor2>(x));
    x = vmax(x, dpp_perm<kDppHalfMirror>(x));
    x = vmax(x, dpp_perm<kDppMirror>(x));
    return vmax(vmax(read_lane(x, 0), read_lane(x, 16)), vmax(read_lane(x, 32), read_lane(x, 48)));
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

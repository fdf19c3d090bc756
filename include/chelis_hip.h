/* MI355X (gfx950) region ABI: the launch surface a fused-DAG emitter binds.
 *
 * In the reference, chelis-backend-hip emits one HIP kernel string per DAG
 * region (crates/chelis-backend-hip/src/kernels.rs) and launches it through
 * hiprtc + hipModuleLaunchKernel on stream 0 (runtime/chelis_hip_runtime.h:
 * 409-485), with matmuls on hipBLAS (runtime/chelis_hip_runtime.h:48-404).
 * Here every region kind is a precompiled gfx950 kernel family behind one
 * `extern "C"` launcher that takes the reference's own device packet
 * (chelis_gpu_tensor). Launchers validate on the host, enqueue on the
 * library's single HIP stream and return without synchronizing; a status
 * other than CHELIS_HIP_OK leaves no work enqueued and sets
 * chelis_hip_last_error(). Which reference kernel each launcher replaces is
 * noted at its declaration.
 *
 * Numerics: every float result is finalized at its dtype with NaN stored as
 * the canonical quiet NaN ([04-NUM-2]); every float sum follows the
 * canonical adjacent-pair tree ([05-OP-30]) bit for bit; RNG, relu, count
 * and max/min selection are bit-exact. Matmuls on the MFMA path are the
 * only results that differ from the canonical tree (by rounding only).
 */
#ifndef CHELIS_HIP_H
#define CHELIS_HIP_H

#include <stdint.h>
#include "chelis_device_descriptor.h"

#ifdef __cplusplus
extern "C" {
#endif

enum {
    CHELIS_HIP_OK = 0,
    CHELIS_HIP_EDOMAIN = 1,      /* invalid shapes, dtypes, rates, axes */
    CHELIS_HIP_EUNSUPPORTED = 2, /* valid request outside the built kernel families */
    CHELIS_HIP_EHIP = 3          /* a HIP runtime call failed */
};

/* ---- context ---- */
const char *chelis_hip_last_error(void);
/* The library's stream on the current device (a hipStream_t), created on
 * first use at default priority. Every launcher enqueues on it. */
void *chelis_hip_stream(void);
int32_t chelis_hip_synchronize(void);
/* Build identification: "gfx950 <git-describe>" style string. */
const char *chelis_hip_build_info(void);
/* Library-wide exact mode (no reference counterpart: the reference has one
 * numeric contract per lane). Non-zero: every result whose primitive the C
 * lane defines bit for bit is computed that way - matmuls (programs
 * included) on the canonical-tree kernels, binary64 softmax rows with the
 * correctly rounded exp and the IEEE division - so results are
 * bit-identical to the C lane (crates/chelis-backend-c). Zero (default):
 * MFMA products and binary64 softmax rows with a faithful exp (within
 * 1 ulp) and one reciprocal per row, within the stated tolerances, as the
 * reference HIP lane's device exp and division are. Affects launches
 * enqueued after the call; returns the previous mode. */
int32_t chelis_hip_set_exact(int32_t on);

/* ---- row regions (last axis; rows contiguous) ----
 * softmax: spec/05 section 4.2 as one region (max_reduce, sub, exp, sum, div),
 * replacing reduce_max + fused_elementwise[Sub,Exp] + reduce_sum + div
 * (kernels.rs:1802,2391,1703) which the reference fences off the device
 * (crates/chelis-ir/src/device_admission.rs:41-68). exp is correctly
 * rounded at f32 and f64, so both are bit-exact with the C lane. */
int32_t chelis_hip_softmax(const chelis_gpu_tensor *x, const chelis_gpu_tensor *y);
/* softmax(where(mask, x * scale, -inf)) over the last axis of a
 * [..., S_q, S_k] score tensor with the causal mask j <= i (spec/05 section
 * 4.7 steps 3-5) when causal != 0; scale is rounded once to the dtype. */
int32_t chelis_hip_scaled_masked_softmax(const chelis_gpu_tensor *x, double scale, int32_t causal,
                                         const chelis_gpu_tensor *y);

/* Causal self-attention in one launch: o = softmax(where(key <= row,
 * (q . k^T) * scale, -inf)) . v over f32 [batch, heads, seq, 64] views, seq
 * a multiple of 64, the head axis contiguous and rows 16-byte aligned; o
 * must not overlap q, k or v. No single counterpart in the reference's C
 * ABI: the fused form of the attention graph of spec/05 section 4.7 (scores
 * matmul, causal where, softmax, P.V) for plans that run the three as one
 * region. Within the binary32 tolerance of the unfused graph, not
 * bit-identical to it. */
int32_t chelis_hip_causal_attention(const chelis_gpu_tensor *q, const chelis_gpu_tensor *k, const chelis_gpu_tensor *v,
                                    double scale, const chelis_gpu_tensor *o);
/* softmax adjoint y * (g - sum(g * y)) (crates/chelis-dag-core/src/grad.rs:2248). */
int32_t chelis_hip_softmax_adjoint(const chelis_gpu_tensor *y, const chelis_gpu_tensor *g,
                                   const chelis_gpu_tensor *dx);
/* layer_norm over the last axis: spec/05 section 4.4 / tier2.rs:1248-1360. */
int32_t chelis_hip_layer_norm(const chelis_gpu_tensor *x, const chelis_gpu_tensor *gamma,
                              const chelis_gpu_tensor *beta, double epsilon, const chelis_gpu_tensor *y);

/* ---- fused elementwise chains (RiscOp::FusedElem, dag.rs:485-524,673-678) ----
 * A step's args index the chain inputs when >= 0, and a previous step k as
 * -(k + 1) (FusedInput::External / FusedInput::PreviousStep). The chain's
 * value is its last step. `imm` is the scalar of CHELIS_FUSED_CONST. */
enum {
    CHELIS_FUSED_ADD = 0, CHELIS_FUSED_SUB, CHELIS_FUSED_MUL, CHELIS_FUSED_DIV,
    CHELIS_FUSED_MAX_ELEM, CHELIS_FUSED_MIN_ELEM, CHELIS_FUSED_NEG, CHELIS_FUSED_RECIP,
    CHELIS_FUSED_EXP, CHELIS_FUSED_LOG, CHELIS_FUSED_SQRT, CHELIS_FUSED_TANH,
    CHELIS_FUSED_ERFC, CHELIS_FUSED_ABS, CHELIS_FUSED_FLOOR, CHELIS_FUSED_CEIL,
    CHELIS_FUSED_ROUND, CHELIS_FUSED_RELU, CHELIS_FUSED_RELU_ADJOINT,
    CHELIS_FUSED_CONST, CHELIS_FUSED_COUNT_
};
#define CHELIS_FUSED_MAX_STEPS 16
#define CHELIS_FUSED_MAX_INPUTS 8
typedef struct {
    uint8_t op;
    uint8_t reserved[3];
    int32_t args[2];
    double imm;
} chelis_fused_step;
typedef struct {
    int32_t n_steps;
    int32_t reserved;
    chelis_fused_step steps[CHELIS_FUSED_MAX_STEPS];
} chelis_fused_chain;
/* kernels.rs:2391 fused_elementwise. Inputs broadcast to `out` by their
 * own strides (stride 0 = expanded axis); out is contiguous. bf16 / f16
 * chains (CHELIS_DTYPE_BF16 / F16) may hold only SUB, MAX_ELEM and MIN_ELEM
 * steps, each computed at binary32 and stored at 16 bits, as the reference
 * admits them (emit.rs:2292-2319, kernels.rs:2274-2373); any other step
 * returns CHELIS_HIP_EUNSUPPORTED. */
int32_t chelis_hip_fused_elementwise(const chelis_fused_chain *chain, const chelis_gpu_tensor *const *inputs,
                                     int32_t n_inputs, const chelis_gpu_tensor *out);

/* ---- reductions over one axis ----
 * kernels.rs:2175 reduce_fused (chain != NULL: the chain's value is the
 * leaf; sum and max only, the reductions fuse.rs:463-487 inlines a chain
 * into) and kernels.rs:1703-2013 reduce_sum/max/min/prod/argmax/argmin
 * (chain == NULL: inputs[0] is the leaf). Sum uses the canonical tree;
 * prod is the C lane's left fold from 1 (crates/chelis-backend-c/src/
 * emit.rs:2551-2561, 8817-8912), NaN-finalized; max/min follow the
 * first-NaN / first-representation rule [05-OP-12/13]; argmax/argmin write
 * i64. `out` has the input shape minus `axis`. */
enum {
    CHELIS_REDUCE_SUM = 0, CHELIS_REDUCE_COUNT = 1, CHELIS_REDUCE_MAX = 2,
    CHELIS_REDUCE_MIN = 3, CHELIS_REDUCE_PROD = 4, CHELIS_REDUCE_ARGMAX = 5,
    CHELIS_REDUCE_ARGMIN = 6
};
int32_t chelis_hip_reduce(int32_t op, const chelis_fused_chain *chain, const chelis_gpu_tensor *const *inputs,
                          int32_t n_inputs, int32_t axis, const chelis_gpu_tensor *out);
/* Allocation-free reduction. No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments, results
 * and statuses as chelis_hip_reduce; the pass partials live in one fixed
 * per-device array of CHELIS_HIP_STATIC_SCRATCH_BYTES (held until the
 * process ends) instead of the library's cached scratch, and the call makes
 * no allocation. A reduction whose partials need more than the array
 * returns CHELIS_HIP_EDOMAIN before enqueueing anything. Every pass writes
 * the partials it later reads, so nothing needs clearing between calls.
 * All calls on a device share its array: calls whose work overlaps in time
 * on one GPU (work on different streams, e.g. a captured graph replayed on
 * another stream beside a direct call) race on it; calls enqueued on the
 * library stream run in order. */
#define CHELIS_HIP_STATIC_SCRATCH_BYTES (8u * 1024u * 1024u)
/* Allocation counters (no counterpart in the reference; for callers and
 * tests that must know an entry allocates nothing): scratch requests
 * served by the library's cache or by a new allocation, and device
 * allocations, each counted since the process started. */
void chelis_hip_allocation_counts(int64_t *scratch_requests, int64_t *device_allocations);
int32_t chelis_hip_reduce_static(int32_t op, const chelis_fused_chain *chain, const chelis_gpu_tensor *const *inputs,
                                 int32_t n_inputs, int32_t axis, const chelis_gpu_tensor *out);
/* kernels.rs:375-557 count: Bool8 -> i64 over one axis. A byte that is not
 * 0/1 raises the reference kernel's error code 1. With error_code, the call
 * synchronizes and stores the code there, as the reference's launch does
 * (emit.rs:4520-4620, one status word per call). With error_code == NULL it
 * returns at once and the code goes to the device's trap channel, to be read
 * once at the end of the caller's entry with chelis_hip_trap_status. */
int32_t chelis_hip_count(const chelis_gpu_tensor *x, int32_t axis, const chelis_gpu_tensor *out,
                         int32_t *error_code);
/* The current device's trap channel: synchronizes the library stream, stores
 * the OR of the codes recorded since the last read (0: none) and clears it.
 * The reference reads its numeric-failure flag after every trapping launch
 * (kernels.rs:21-32, emit.rs:5185-5240); this channel lets an entry read it
 * once, after its last launch. */
int32_t chelis_hip_trap_status(int32_t *code);

/* ---- comparison, logical, where ----
 * One launch per node, as the reference HIP lane's kernels: comparison
 * (kernels.rs:1266-1300) of two operands of one dtype to Bool8 - IEEE
 * comparison of the semantic values for f32 / f64 / bf16 / f16 (any NaN
 * false, neq true; signed zeros equal), exact order for i8..i64, eq / neq
 * only for bool ([05-OP-36]); logical and / or / not on Bool8 bytes, a byte
 * true when nonzero (kernels.rs:1303-1336; b is ignored for not); where
 * (kernels.rs:1338-1380): the selected branch's stored bits, any dtype.
 * Operands broadcast to `out` by their own strides (stride 0 = expanded
 * axis); out is contiguous. No failure is possible. */
enum {
    CHELIS_CMP_CMPLT = 0, CHELIS_CMP_LT = 1, CHELIS_CMP_EQ = 2, CHELIS_CMP_NEQ = 3,
    CHELIS_CMP_GT = 4, CHELIS_CMP_GTE = 5, CHELIS_CMP_LTE = 6
};
int32_t chelis_hip_compare(int32_t kind, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                           const chelis_gpu_tensor *out);
enum { CHELIS_LOGICAL_AND = 0, CHELIS_LOGICAL_OR = 1, CHELIS_LOGICAL_NOT = 2 };
int32_t chelis_hip_logical(int32_t kind, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                           const chelis_gpu_tensor *out);
int32_t chelis_hip_where(const chelis_gpu_tensor *cond, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                         const chelis_gpu_tensor *out);

/* ---- extrema cotangent ----
 * kernels.rs:1030-1134 (RiscOp::ExtremaAdjoint{kind, operand}, [05-OP-40]):
 * out = g where `operand` was selected by max_elem / min_elem of (a, b),
 * +0 elsewhere. max selects a when a is NaN, or when b is not NaN and
 * a >= b (min: a <= b). f32, f64, bf16, f16 (16-bit operands compare their
 * decoded values; the cotangent keeps its stored bits). */
enum { CHELIS_EXTREMA_MAX = 0, CHELIS_EXTREMA_MIN = 1 };
enum { CHELIS_EXTREMA_LEFT = 0, CHELIS_EXTREMA_RIGHT = 1 };
int32_t chelis_hip_extrema_adjoint(int32_t kind, int32_t operand, const chelis_gpu_tensor *a,
                                   const chelis_gpu_tensor *b, const chelis_gpu_tensor *g,
                                   const chelis_gpu_tensor *out);

/* ---- checked casts, checked integer arithmetic, gather ----
 * Failures follow [04-NUM-9]: a failing element stores zero and the launch
 * reports the lowest-index failing element ([04-NUM-15]) with its kind and
 * the rendered trap line. With `failure` non-NULL the call waits for its
 * own result and fills *failure (kind 0: none), as the reference reads its
 * numeric-failure record after a trapping launch (emit.rs:5185-5240). With
 * `failure` NULL it returns at once and records into the device's deferred
 * record, which chelis_hip_take_numeric_failure reads once after a run of
 * launches: the earliest launch that failed, at its lowest failing index.
 *
 * cast: [04-NUM-14]'s checked cast between f32, f64, bf16, f16, i8, i16,
 * i32, i64 and bool, with the C lane's conversions
 * (crates/chelis-backend-c/src/host_emit.rs:1700-2120; the reference HIP
 * lane's cast kernels are kernels.rs:1382, 2489, 2521): equal dtypes keep the
 * stored bits; a float to an integer fails `domain` unless finite and
 * integral, then `overflow` outside the range; an integer or bool to an
 * integer fails `overflow` outside the range; to bool anything but 0 / 1
 * fails `domain`; to a float, one rounding to nearest even from the exact
 * source value, NaN to the canonical quiet NaN. Trap line
 * `numeric trap: <kind> in cast at <target>`.
 *
 * integer_elementwise: i8 / i16 / i32 / i64 at the operand width
 * (crates/chelis-numeric-core/src/dtype_semantics.rs:930-1030): add, sub,
 * mul, neg and abs fail `overflow` outside the range; floor_div, trunc_div
 * and mod fail `division by zero` on a zero divisor, floor_div and
 * trunc_div `overflow` on MIN / -1; max_elem / min_elem never fail. The
 * reference HIP lane checks sub and abs only (kernels.rs:769-810, 1434) and
 * has no mod (emit.rs:2574); this build checks every op as the C lane does.
 * b is ignored for neg and abs. Trap line `numeric trap: <kind> in <op> at
 * <dtype>`. The bitwise ops ([05-OP-47], RiscOp::Bitwise, the reference HIP
 * lane's binary_bitwise_typed, kernels.rs:687-760): bitand / bitor / bitxor
 * on the w-bit two's complement; shl and shr take b as the count - a count
 * at or above w gives 0 (shr of a negative value: -1), shr extends the sign
 * - and a negative count fails `domain` with the C lane's line
 * `shift amount must be non-negative, got <count>` ([04-NUM-13],
 * crates/chelis-runtime/include/chelis_runtime.h:297-330) as the message.
 *
 * gather: RiscOp::Gather{axis, batch_rank} (crates/chelis-dag-core/src/
 * dag.rs:1349-1356) with the reference's geometry (emit.rs:3807-3900,
 * kernels.rs:2557-2597): out = values[..axis] ++ indices[batch_rank..] ++
 * values[axis+1..], the first batch_rank axes of values and indices paired;
 * element (b, j, d) reads values at index indices[batch of b, j] on `axis`.
 * Any dtype of values (the reference admits f32 / f64), i32 or i64 indices,
 * strided views of either. An index outside [0, extent) fails `domain`
 * (`numeric trap: domain in gather at i64`); paired batch extents that
 * differ return CHELIS_HIP_EDOMAIN with that line before any launch. */
typedef struct {
    int64_t index;     /* row-major index of the first failing element, -1 when none */
    int32_t kind;      /* 0 none, 1 overflow, 2 domain, 3 division by zero */
    int32_t reserved;
    char message[96];  /* the trap line, e.g. "numeric trap: overflow in add at i64"; "" when none */
} chelis_hip_numeric_failure;
int32_t chelis_hip_cast(const chelis_gpu_tensor *x, const chelis_gpu_tensor *out,
                        chelis_hip_numeric_failure *failure);
enum {
    CHELIS_INT_ADD = 0, CHELIS_INT_SUB = 1, CHELIS_INT_MUL = 2, CHELIS_INT_FLOOR_DIV = 3,
    CHELIS_INT_TRUNC_DIV = 4, CHELIS_INT_MOD = 5, CHELIS_INT_MAX_ELEM = 6, CHELIS_INT_MIN_ELEM = 7,
    CHELIS_INT_NEG = 8, CHELIS_INT_ABS = 9, CHELIS_INT_BITAND = 10, CHELIS_INT_BITOR = 11,
    CHELIS_INT_BITXOR = 12, CHELIS_INT_SHL = 13, CHELIS_INT_SHR = 14
};
int32_t chelis_hip_integer_elementwise(int32_t op, const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                                       const chelis_gpu_tensor *out, chelis_hip_numeric_failure *failure);
int32_t chelis_hip_gather(const chelis_gpu_tensor *values, const chelis_gpu_tensor *indices, int32_t axis,
                          int32_t batch_rank, const chelis_gpu_tensor *out, chelis_hip_numeric_failure *failure);
/* cumsum: RiscOp::Cumsum{axis, direction} ([05-OP-33]; the reference HIP
 * lane's ordered_scan, kernels.rs:2793, with the C lane's accumulation,
 * crates/chelis-runtime/src/lib.rs:7020-7105): an inclusive scan along
 * `axis`, from the end when `reverse` (the decreasing direction). The first
 * leaf is the first prefix; each later one adds the leaf at the accumulator
 * width - binary32 for bf16 / f16, i32 for i8 / i16 (whose result is i32),
 * the dtype otherwise - and each prefix is stored at the result dtype, NaN
 * canonical. An integer prefix out of range fails `overflow`
 * (`numeric trap: overflow in cumsum at <result dtype>`); the failure's
 * index is then the prefix's place in the scan's evaluation order (line by
 * line: ((o * inner + j) * n + step)), the order the C lane traps in. */
int32_t chelis_hip_cumsum(const chelis_gpu_tensor *x, int32_t axis, int32_t reverse, const chelis_gpu_tensor *out,
                          chelis_hip_numeric_failure *failure);
/* pad: RiscOp::Pad{padding, fill} (crates/chelis-dag-core/src/dag.rs:1202;
 * the reference HIP lane's pad_typed, kernels.rs:1587-1637). out has x's
 * rank and dtype; lo[a] elements come before x on axis a, and out's extent
 * leaves out->shape[a] - lo[a] - x->shape[a] >= 0 after it. Every element
 * outside x is fill_bits' low dtype-width bytes (a float's stored bits, an
 * integer's two's complement). Any strides on either side (the output's
 * elements must not overlap); rank <= 8. */
int32_t chelis_hip_pad(const chelis_gpu_tensor *x, const int64_t *lo, uint64_t fill_bits,
                       const chelis_gpu_tensor *out);
/* scatter: RiscOp::ScatterAdd{axis, batch_rank} when `add`, else
 * RiscOp::Scatter{axis, batch_rank} (crates/chelis-dag-core/src/dag.rs:
 * 1360-1384), replacing the reference HIP lane's scatter_add (atomics) and
 * single-thread scatter_replace (kernels.rs:2599-2716) with the C lane's
 * results (crates/chelis-backend-c/src/emit.rs:7382-7470, 7842-7990). out
 * has the target's shape; updates the gathered shape target[..axis] ++
 * indices[batch_rank..] ++ target[axis+1..] (else CHELIS_HIP_EDOMAIN with
 * `numeric trap: domain in scatter at i64`). Update u goes where the gather
 * of the same geometry would read. Replace: each cell takes its last update
 * in row-major position (the last write). Add: each targeted cell is the
 * canonical pair tree over [its target value, its updates in ascending
 * position] at the operand width (bf16 / f16 rounded at every node, the
 * total NaN-canonical); any dtype but bool. An index outside the axis fails
 * `domain` at the update's position (`numeric trap: domain in scatter at
 * i64`, or `scatter_replace`); an integer node outside the width fails
 * `overflow` (`numeric trap: overflow in scatter at <dtype>`), its index the
 * update count plus the destination's row-major index. Operands may be
 * strided; out contiguous. At most 2^31 - 1 updates.
 *
 * scatter_elements: RiscOp::ScatterElements{axis} (dag.rs:1386-1404;
 * kernels.rs:2718-2765): indices and updates share a shape and every
 * operand the data's rank, no index extent off the axis above the data's
 * (crates/chelis-abi/src/metadata.rs:831-846); the update at coordinates c
 * goes to c with c[axis] = indices[c], the last write winning. Failures as
 * scatter's, named scatter_elements. */
int32_t chelis_hip_scatter(int32_t add, const chelis_gpu_tensor *target, const chelis_gpu_tensor *indices,
                           const chelis_gpu_tensor *updates, int32_t axis, int32_t batch_rank,
                           const chelis_gpu_tensor *out, chelis_hip_numeric_failure *failure);
int32_t chelis_hip_scatter_elements(const chelis_gpu_tensor *data, const chelis_gpu_tensor *indices,
                                    const chelis_gpu_tensor *updates, int32_t axis, const chelis_gpu_tensor *out,
                                    chelis_hip_numeric_failure *failure);
/* Waits for the library stream, then reads and clears the current device's
 * deferred failure record (kind 0: none). */
int32_t chelis_hip_take_numeric_failure(chelis_hip_numeric_failure *failure);

/* ---- keyed RNG ([05-RNG-1/2], [05-OP-8], [05-OP-37]) ----
 * uniform_like: kernels.rs:1672. dropout / replay: the C lane's semantics
 * (crates/chelis-backend-c/src/emit.rs:6139-6220); the reference HIP lane
 * rejects them (crates/chelis-backend-hip/src/emit.rs:2763-2778). A rate
 * outside [0, 1) returns CHELIS_HIP_EDOMAIN with the reference's trap text
 * `numeric trap: domain in dropout at f32|f64` as the last error. */
int32_t chelis_hip_uniform_like(uint64_t key, double low, double high, const chelis_gpu_tensor *out);
int32_t chelis_hip_dropout(uint64_t key, const chelis_gpu_tensor *x, double rate, const chelis_gpu_tensor *y);
int32_t chelis_hip_dropout_replay(uint64_t key, const chelis_gpu_tensor *g, double rate,
                                  const chelis_gpu_tensor *dx);
/* The drop test unit(key, i) < rate at the dtype (the unit (word >> 11) *
 * 2^-53 taken to the dtype, rounded to nearest for f32) as the integer test
 * (word >> 11) < cut the kernels run: the least m in [0, 2^53] whose unit
 * is not below the rate. No counterpart in the reference (its C lane
 * compares the units); exported so the equivalence can be checked. */
uint64_t chelis_hip_dropout_cut(double rate, int32_t dtype);

/* ---- activations ----
 * gelu: spec/05 section 3.3's Phi graph (fenced on the reference HIP
 * lane): bit for bit in the exact mode (chelis_hip_set_exact); in the
 * default mode binary32 is evaluated directly as x Phi(x), within 1e-6
 * relative of the graph (binary64 is the graph in both). relu / relu
 * adjoint: kernels.rs:1136-1196, and for bf16 / f16 operands
 * kernels.rs:1196-1260 (stored bits selected). */
int32_t chelis_hip_gelu(const chelis_gpu_tensor *x, const chelis_gpu_tensor *y);
int32_t chelis_hip_relu(const chelis_gpu_tensor *x, const chelis_gpu_tensor *y);
int32_t chelis_hip_relu_adjoint(const chelis_gpu_tensor *x, const chelis_gpu_tensor *g,
                                const chelis_gpu_tensor *dx);

/* ---- matmul dispatch (BlasMatmul, dag.rs:1338-1352; hipBLAS wrappers
 * chelis_hip_runtime.h:48-404) ----
 * c[..., M, N] = a[..., M, K] . b[..., K, N] with any element strides on a
 * and b (a transposed operand is a stride swap, never a copy; up to two
 * batch axes broadcast numpy-style, an extent-1 axis by stride 0; a rank-1
 * a is a row [1, K] and a rank-1 b a column [K, 1], their axis dropped from
 * c) and c any non-overlapping view. Dense shapes run on MFMA
 * (v_mfma_f32_16x16x4_f32 / v_mfma_f64_16x16x4_f64); short K (<= 32), GEMV
 * (M or N == 1) and skinny shapes (min(M, N) < 16, or <= 64 in f64) run on
 * VALU kernels whose K sum is the canonical tree, bit-exact with the C lane.
 * `flags` = CHELIS_MATMUL_EXACT forces the canonical-tree kernels on every
 * shape. bf16 / f16 operands (all three of one dtype) run on
 * v_mfma_f32_16x16x32_bf16 / _f16 with a binary32 accumulator and a 16-bit
 * result (the reference's hipblasGemmEx with HIPBLAS_COMPUTE_32F,
 * runtime/chelis_hip_runtime.h:92-170); with CHELIS_MATMUL_EXACT they are
 * widened, run through the binary32 canonical tree and encoded once,
 * bit-exact with the C lane. */
#define CHELIS_MATMUL_EXACT 1
int32_t chelis_hip_matmul(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, const chelis_gpu_tensor *c,
                          int32_t flags);
/* matmul with a fused epilogue, applied per element of the f32/f64 result
 * in graph order: v = mm; if bias: v = v + bias[n]; act 1: v = relu(v),
 * act 2: v = gelu(v); if residual: v = residual + v. Each step finalizes
 * at the dtype, so the bits equal the unfused graph's. `bias` is [N], shared
 * by every batch entry, or [batch..., N] with the result's batch axes (one
 * bias row per batch entry, e.g. a stack of projections sharing one input).
 * b may carry batch axes as in chelis_hip_matmul. f32 / f64 only: the
 * reference gives 16-bit matmuls no epilogue (CHELIS_HIP_EUNSUPPORTED). */
enum { CHELIS_ACT_NONE = 0, CHELIS_ACT_RELU = 1, CHELIS_ACT_GELU = 2 };
int32_t chelis_hip_linear(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, const chelis_gpu_tensor *bias,
                          int32_t activation, const chelis_gpu_tensor *residual, const chelis_gpu_tensor *c,
                          int32_t flags);

#ifdef __cplusplus
}
#endif
#endif

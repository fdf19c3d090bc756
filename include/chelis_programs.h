/* Program entries: what the HIP backend generates for the configuration
 * programs, in the reference's generated-entry form.
 *
 * The reference emitter writes one `{f}_device` per compiled function
 * (crates/chelis-backend-hip/src/emit.rs:838-964; signature lib.rs:116-118,
 * normative spec/11-ffi.md:144-156): inputs are borrowed device owners on
 * the current device, each output is a fresh owned contiguous tensor the
 * caller releases with chelis_device_tensor_release, and the call returns
 * after the device work is done. Invalid arity or shapes trap `domain`
 * (stderr, exit status 1) like the reference entry.
 *
 * Each `{f}_device` has a `chelis_prog_{f}` companion that takes device
 * packets for inputs AND outputs, enqueues the whole program on the
 * library stream and returns a CHELIS_HIP_* status without synchronizing:
 * the form a caller that owns its buffers (or times the program) uses.
 *
 * Region kernels are the ones in chelis_hip.h; the programs below are the
 * BASELINE configuration programs, restated from their descriptions:
 *   linreg_step       X f64[n,d], w[d], y[n] -> grad[d], loss[]
 *                     r = X.w - y; grad = X^T.r / n; loss = mean(r*r)
 *   transformer_block x f32[B,S,D] + 16 parameters (ln1_g ln1_b Wq bq Wk bk
 *                     Wv bv Wo bo ln2_g ln2_b W1 b1 W2 b2) -> y[B,S,D];
 *                     pre-LN, causal multi-head attention with 64-wide
 *                     heads (D/64 heads), GELU FFN, eps 1e-5
 *   mlp_train_step    x f32[B,I], onehot[B,O], w1[I,H], b1[H], w2[H,O],
 *                     b2[O], key (KEY, rank 0) -> loss[], w1', b1', w2', b2';
 *                     relu, keyed dropout rate 0.1, softmax cross-entropy
 *                     (mean over the batch), reverse mode, SGD lr 0.01
 */
#ifndef CHELIS_PROGRAMS_H
#define CHELIS_PROGRAMS_H

#include "chelis_device_owner.h"
#include "chelis_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

void linreg_step_device(const chelis_device_tensor_owner *const *inputs, chelis_device_rank n_in,
                        chelis_device_tensor_owner **outputs, chelis_device_rank n_out);
void transformer_block_device(const chelis_device_tensor_owner *const *inputs, chelis_device_rank n_in,
                              chelis_device_tensor_owner **outputs, chelis_device_rank n_out);
void mlp_train_step_device(const chelis_device_tensor_owner *const *inputs, chelis_device_rank n_in,
                           chelis_device_tensor_owner **outputs, chelis_device_rank n_out);

/* The generated host-tensor entries `{f}` (emit.rs:667-808, header
 * lib.rs:116-118): host tensors in, new host tensors out (chelis_alloc,
 * written under a write lease, released by the caller with
 * chelis_tensor_release); a wrong input or output count prints
 * "{f}: expected N inputs, got M" and aborts; the device is synchronized
 * before the call returns. */
void linreg_step(chelis_tensor **inputs, int n_in, chelis_tensor **outputs, int n_out);
void transformer_block(chelis_tensor **inputs, int n_in, chelis_tensor **outputs, int n_out);
void mlp_train_step(chelis_tensor **inputs, int n_in, chelis_tensor **outputs, int n_out);

int32_t chelis_prog_linreg_step(const chelis_gpu_tensor *const *inputs, int32_t n_in,
                                const chelis_gpu_tensor *const *outputs, int32_t n_out);
int32_t chelis_prog_transformer_block(const chelis_gpu_tensor *const *inputs, int32_t n_in,
                                      const chelis_gpu_tensor *const *outputs, int32_t n_out);
int32_t chelis_prog_mlp_train_step(const chelis_gpu_tensor *const *inputs, int32_t n_in,
                                   const chelis_gpu_tensor *const *outputs, int32_t n_out);

/* The exact mode of chelis_hip_set_exact (chelis_hip.h) under its first
 * name: non-zero routes every matmul (programs included) through the
 * canonical-tree kernels, so whole programs are bit-exact with the C lane
 * except for leaves that are not correctly rounded on the device (binary64
 * log, erfc, tanh). Returns the previous mode. */
int32_t chelis_hip_set_exact_matmul(int32_t on);

#ifdef __cplusplus
}
#endif
#endif

/* Runtime C ABI subset used by generated entries and the device owner.
 *
 * Replaces the tensor / metadata-plan part of the reference runtime
 * (crates/chelis-runtime/include/chelis_runtime.h, Rust staticlib
 * crates/chelis-runtime/src/lib.rs); names, layouts and trap behaviour are
 * the reference's. Implemented in C++ in chelis_amd/csrc/runtime.cpp.
 * Strings, lists, dicts, CSV, mmap and host I/O are not on the tensor path
 * and are not provided. */
#ifndef CHELIS_RUNTIME_H
#define CHELIS_RUNTIME_H

#include <stdbool.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "chelis_runtime_dtype.h"

typedef struct chelis_tensor chelis_tensor;
typedef struct chelis_tensor_write chelis_tensor_write;

/* chelis_runtime.h:27-28 */
typedef struct { chelis_dtype dtype; uint8_t reserved[7]; uint64_t bits; } chelis_scalar;
typedef struct { uint64_t bits; } chelis_key;
#include "chelis_runtime_views.h"

#ifdef __cplusplus
extern "C" {
#endif

/* chelis_runtime.h:39: a zero-filled contiguous host tensor, refcount 1. */
chelis_tensor *chelis_alloc(int32_t rank, const int64_t *shape, chelis_dtype dtype);
/* chelis_runtime.h:41: borrows caller storage of at least the logical bytes. */
chelis_tensor *chelis_tensor_entry_borrow(int32_t rank, const int64_t *shape, chelis_dtype dtype,
                                          const void *data, int64_t byte_capacity);
/* chelis_runtime.h:42-43 */
void chelis_tensor_retain(const chelis_tensor *tensor);
void chelis_tensor_release(const chelis_tensor *tensor);
/* chelis_runtime.h:45 */
chelis_read_view chelis_tensor_read_view(const chelis_tensor *tensor);
/* chelis_runtime.h:47-49: one write lease at a time. */
chelis_tensor_write *chelis_tensor_begin_write(chelis_tensor *tensor);
chelis_write_view chelis_tensor_write_view(const chelis_tensor_write *guard);
void chelis_tensor_end_write(chelis_tensor_write *guard);
/* chelis_runtime.h:56 */
int64_t chelis_dtype_size(chelis_dtype dtype);
/* chelis_runtime.h:328-332 */
chelis_scalar chelis_scalar_from_bits(chelis_dtype dtype, uint64_t bits);
chelis_key chelis_key_from_seed(int64_t seed);
/* chelis_runtime.h:350-352 */
int32_t chelis_tensor_rank(const chelis_tensor *tensor);
int64_t chelis_tensor_shape(const chelis_tensor *tensor, int32_t axis);
int64_t chelis_tensor_numel(const chelis_tensor *tensor);

/* chelis_runtime.h:367-378: checked metadata only, no payload. Every
 * invalid request traps `numeric trap: domain|overflow in metadata_plan at i64`. */
typedef struct chelis_metadata_plan chelis_metadata_plan;
chelis_metadata_plan *chelis_metadata_plan_new(chelis_scalar rank, const chelis_scalar *shape, chelis_scalar exemplar);
chelis_metadata_plan *chelis_metadata_plan_view(chelis_scalar rank, const chelis_scalar *shape, const chelis_scalar *strides,
                                                chelis_scalar exemplar, chelis_scalar byte_capacity);
int32_t chelis_metadata_plan_rank(const chelis_metadata_plan *plan);
const int64_t *chelis_metadata_plan_shape(const chelis_metadata_plan *plan);
const int64_t *chelis_metadata_plan_strides(const chelis_metadata_plan *plan);
int64_t chelis_metadata_plan_count(const chelis_metadata_plan *plan);
int64_t chelis_metadata_plan_byte_count(const chelis_metadata_plan *plan);
int64_t chelis_metadata_plan_byte_offset(const chelis_metadata_plan *plan, chelis_scalar linear_index);
chelis_dtype chelis_metadata_plan_dtype(const chelis_metadata_plan *plan);
void chelis_metadata_plan_check_capacity(const chelis_metadata_plan *plan, chelis_scalar byte_capacity);
void chelis_metadata_plan_release(chelis_metadata_plan *plan);

/* chelis_runtime.h:785: host tensors here are always contiguous, so this
 * returns the input retained. */
chelis_tensor *chelis_contiguous(const chelis_tensor *tensor);

#ifdef __cplusplus
}
#endif

/* chelis_runtime.h:73-82,127-130: a trap is a process failure at the lane
 * boundary: message to stderr, both streams flushed, exit status 1. */
static inline void chelis_flush_and_exit_trap(void) {
    (void)fflush(stdout);
    (void)fflush(stderr);
    exit(1);
}
static inline void chelis_numeric_trap(const char *message) {
    fprintf(stderr, "%s\n", message);
    chelis_flush_and_exit_trap();
}

#endif

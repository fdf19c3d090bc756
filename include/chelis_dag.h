/* The DAG front end: a lowered or fused Chelis RISC DAG, in the reference's
 * serde JSON wire form, run on gfx950 through this library's region
 * launchers.
 *
 * In the reference, `chelis build --target hip` fuses the DAG
 * (crates/chelis-dag-core/src/fuse.rs:32), lowers it to HIP source with one
 * kernel string per fused node (codegen_hip, crates/chelis-backend-hip/src/
 * lib.rs:104-167; HipEmitter::emit_dag, emit.rs:488-964) and compiles that.
 * Here the same DAG is read as JSON (the form serde_json::to_string(&dag)
 * writes, crates/chelis-dag-core/src/dag.rs:2364-2400,2913-2919), its
 * lowered patterns become single region launches (a matmul with its bias /
 * activation / residual epilogue, softmax, causal masked softmax, softmax
 * adjoint, layer norm, GELU), the rest is grouped by fuse.rs's chain rules,
 * and intermediates share one planned workspace.
 *
 * Errors: a NULL result or a status other than CHELIS_HIP_OK, with
 * chelis_hip_last_error() describing it (the node and op a plan cannot run
 * are named, as the reference's Unsupported diagnostics do). */
#ifndef CHELIS_DAG_H
#define CHELIS_DAG_H

#include <stdint.h>
#include "chelis_device_descriptor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct chelis_dag_program chelis_dag_program;

/* Reads and plans a DAG; host work only (constants reach a device on the
 * first run there). The inputs are the DAG's Load names in first-appearance
 * order (a repeated name is one input); the outputs its Store nodes, then
 * its roots, each node once (the reference's output specs,
 * crates/chelis-backend-hip/src/emit.rs:5881-5933).
 *
 * Run-time extents: a dimension declared as Named(name, None), or an
 * RtDim Sym / InputAxis extent, is a symbol bound when the program runs
 * from the first input axis that declares it; every other declaring axis
 * must agree. One compiled program runs at any binding. */
chelis_dag_program *chelis_dag_compile(const char *json, int64_t length);
void chelis_dag_release(chelis_dag_program *program);
/* Enqueues the program on the library stream (chelis_hip_stream()) over
 * caller-owned device packets; returns without synchronizing. Input packets
 * may be any strided views of the declared shapes and dtypes; outputs have
 * the shapes chelis_dag_output_shape reports for these inputs. */
int32_t chelis_dag_run(chelis_dag_program *program, const chelis_gpu_tensor *const *inputs, int32_t n_in,
                       const chelis_gpu_tensor *const *outputs, int32_t n_out);

/* The program's numeric mode (no counterpart in the reference, which has
 * one numeric contract per lane): 1 exact (every primitive the C lane
 * defines bit for bit computed that way), 0 default, -1 (the initial
 * setting) the library-wide chelis_hip_set_exact mode, read once at the
 * start of each run. Every launch of one run uses one mode. Returns the
 * previous setting. */
int32_t chelis_dag_set_exact(chelis_dag_program *program, int32_t mode);
int32_t chelis_dag_input_count(const chelis_dag_program *program);
int32_t chelis_dag_output_count(const chelis_dag_program *program);
/* output == 0: input slot `index` (its Load's name); 1: output slot (a
 * Store's name, else "root<index>" with the root's position). */
const char *chelis_dag_label(const chelis_dag_program *program, int32_t output, int32_t index);
/* The declared type; a run-time extent is reported as -1. */
int32_t chelis_dag_type(const chelis_dag_program *program, int32_t output, int32_t index, int32_t *rank,
                        int64_t *shape, int32_t shape_capacity, int32_t *dtype);
/* Output `index`'s shape for these inputs (their run-time extents bound as
 * chelis_dag_run binds them); host work only. */
int32_t chelis_dag_output_shape(const chelis_dag_program *program, const chelis_gpu_tensor *const *inputs,
                                int32_t n_in, int32_t index, int32_t *rank, int64_t *shape, int32_t shape_capacity);
/* The run-time extents, in binding order (the reference's symbolic_dims). */
int32_t chelis_dag_symbol_count(const chelis_dag_program *program);
const char *chelis_dag_symbol_name(const chelis_dag_program *program, int32_t index);
/* Workspace plus constant pool bytes one run needs on a device (the
 * reference's peak_device_bytes_estimate, memory.rs:130-155); -1 when a
 * run-time extent sizes it. _at evaluates it for extents given in binding
 * order (HipCodegenResult::peak_device_bytes_at, lib.rs:67-77). */
int64_t chelis_dag_peak_device_bytes(const chelis_dag_program *program);
int64_t chelis_dag_peak_device_bytes_at(const chelis_dag_program *program, const int64_t *values, int32_t n);
int64_t chelis_dag_launch_count(const chelis_dag_program *program);
/* One line per launch: index, region kind, result node, input nodes. */
const char *chelis_dag_describe(const chelis_dag_program *program);

/* fuse.rs on its own: the DAG after greedy chain fusion, as JSON in the same
 * wire form (a thread-local string, valid until the next call). */
const char *chelis_dag_fuse(const char *json, int64_t length);

/* ---- codegen surface: the reference's HipCodegenResult
 * (crates/chelis-backend-hip/src/lib.rs:32-53) ----
 * codegen_hip(dag, func_name) writes host C++ defining
 *   void {f}(chelis_tensor **, int, chelis_tensor **, int);
 *   void {f}_device(const chelis_device_tensor_owner *const *, chelis_device_rank,
 *                   chelis_device_tensor_owner **, chelis_device_rank);
 * with the reference's entry contracts (emit.rs:667-808, 838-964), built by
 * compiling it with compile_flags and linking link_flags (this library in
 * place of -lhiprtc -lhipblas). */
typedef struct chelis_hip_codegen_result chelis_hip_codegen_result;
chelis_hip_codegen_result *chelis_codegen_hip(const char *json, int64_t length, const char *func_name);
void chelis_codegen_release(chelis_hip_codegen_result *result);
const char *chelis_codegen_c_source(const chelis_hip_codegen_result *result);
const char *chelis_codegen_h_header(const chelis_hip_codegen_result *result);
/* which: 0 compile flags, 1 link flags, 2 input labels, 3 output labels,
 * 4 symbolic dims */
int32_t chelis_codegen_list_count(const chelis_hip_codegen_result *result, int32_t which);
const char *chelis_codegen_list_item(const chelis_hip_codegen_result *result, int32_t which, int32_t index);
const char *chelis_codegen_peak_device_bytes_formula(const chelis_hip_codegen_result *result);
/* -1 when an extent is known only at run time */
int64_t chelis_codegen_peak_device_bytes_estimate(const chelis_hip_codegen_result *result);

/* ---- the rest of the reference's build-side surface ----
 * prepare_dag_for_codegen (crates/chelis-backend-hip/src/lib.rs:173-227):
 * the BLAS selection before codegen - each lowered matmul
 * [Cast](Sum(Mul(Expand(a), Expand(b)))) the reference's recognizer takes
 * (crates/chelis-ir-core/src/specialize.rs:150-226,623-793) becomes one
 * BlasMatmul node - written back in the wire form (a thread-local string,
 * valid until the next call). No Realize copies are inserted: this
 * library's matmul reads strided operands. Idempotent. */
const char *chelis_prepare_dag_for_codegen(const char *json, int64_t length);
/* TENSOR_CAPABLE_PRIMS (lib.rs:10-18): the dtype ids of the primitive types
 * the tensor path realizes; returns their count. */
int32_t chelis_hip_tensor_capable_prims(const chelis_dtype **prims);
/* runtime_dir() (lib.rs:81-83): the directory of the headers generated
 * code includes (this library's include/), as an absolute path. */
const char *chelis_hip_runtime_dir(void);

/* codegen_hip_host_program (lib.rs:229-300): of a host program's tensor
 * helpers (name and DAG each, the wrapper's helper manifest), every helper
 * whose DAG holds a Count becomes its own HIP translation unit through
 * chelis_codegen_hip under its own name; the others keep their C-host
 * disposition and are not listed. The scalar / container host wrapper
 * itself is the C backend's output, which this library does not produce;
 * it declares each listed helper as an external symbol. */
typedef struct chelis_hip_host_program_result chelis_hip_host_program_result;
chelis_hip_host_program_result *chelis_codegen_hip_host_program(int32_t n_helpers, const char *const *names,
                                                                const char *const *dags, const int64_t *lengths);
void chelis_host_program_release(chelis_hip_host_program_result *result);
int32_t chelis_host_program_helper_count(const chelis_hip_host_program_result *result);
const char *chelis_host_program_helper_name(const chelis_hip_host_program_result *result, int32_t index);
/* owned by `result` */
const chelis_hip_codegen_result *chelis_host_program_helper(const chelis_hip_host_program_result *result,
                                                            int32_t index);

#ifdef __cplusplus
}
#endif
#endif

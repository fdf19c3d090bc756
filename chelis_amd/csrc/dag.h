// The DAG front end: reads a lowered or fused Chelis RISC DAG in the
// reference's serde JSON shape, forms launch regions, plans their memory and
// runs them through this library's region launchers (include/chelis_dag.h).
//
// Pipeline (each stage in its own file):
//   dag_json.cpp    JSON text <-> Json values
//   dag_read.cpp    Json -> Graph (the reference's Dag / DagNode / RiscOp
//                   wire form, crates/chelis-dag-core/src/dag.rs:835-1352,
//                   2364-2400, 2913-2919) and Graph -> JSON
//   dag_fuse.cpp    fuse.rs's greedy single-consumer chains and the
//                   reduction-inlined chain set (crates/chelis-dag-core/src/
//                   fuse.rs:32-487), plus the inverse (a FusedElem back to
//                   its primitive nodes) so patterns see one form
//   dag_plan.cpp    region formation (matmul + epilogue, softmax, masked
//                   softmax, softmax adjoint, layer norm, GELU, dropout,
//                   reductions, chains), output layouts and the slot plan
//   dag_exec.cpp    packets at run time and the launches; the C ABI
//   dag_codegen.cpp host source for `{f}` / `{f}_device` over the same plan
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "chelis_hip.h"

namespace chelis {
namespace dag {

// ---------------------------------------------------------------- JSON
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool boolean = false;
    std::string text;  // number spelling or string value
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> fields;

    const Json *get(const char *key) const;
    bool is_int() const;
    int64_t as_int() const;  // caller checks is_int()
    double as_double() const;
};
// Parses `n` bytes; on failure returns false and describes the position.
bool parse_json(const char *s, size_t n, Json *out, std::string *error);
void write_json(const Json &v, std::string *out);
std::string json_quote(const std::string &s);

// ---------------------------------------------------------------- IR
enum class Prim : uint8_t { F32, F64, F16, Bf16, Int8, Int16, Int32, Int64, Bool, Key, Other };
const char *prim_name(Prim p);
int64_t prim_width(Prim p);
chelis_dtype prim_dtype(Prim p);
bool prim_is_float(Prim p);
bool is_integer(Prim p);  // i8, i16, i32, i64

enum class Op : uint8_t {
    // leaves
    Load, Const, Iota,
    // elementwise ops fuse.rs folds into chains (fused_step_op, fuse.rs:98-127)
    Add, Sub, Mul, Div, Pow, FloorDiv, TruncDiv, MaxElem, MinElem, Neg, Recip, Exp, Log, Sin, Sqrt, Cos, Tan,
    Atan, Tanh, Erf, Erfc, Abs, Floor, Ceil, Round,
    // elementwise ops that stay their own node
    Relu, ReluAdjoint, Where, Compare, Dropout, DropoutReplay, Cast, Logical, Mod,
    // sparse selection along one axis
    Gather,
    // the extrema cotangent; keyed draws and emission-time key derivations
    ExtremaAdjoint, UniformLike, KeyFromSeed, SplitKey, FoldIn,
    // the ordered inclusive scan
    Cumsum,
    // two's-complement bitwise ops and shifts (code: the kind)
    Bitwise,
    // movement with bounds: pad (a materialized copy), shrink and stride
    // (views)
    Pad, Shrink, Stride,
    // sparse writes: target, indices, updates (axis, batch_rank)
    ScatterAdd, Scatter, ScatterElements,
    // a literal tensor; the release of a value (no data moves)
    ConstTensor, Drop,
    // reductions over one axis
    Sum, MaxReduce, MinReduce, ProdReduce, Argmax, Argmin, Count, Softmax,
    // movement
    Expand, Permute, Reshape, Realize, Copy,
    // fused and specialized forms
    FusedElem, BlasMatmul,
    // outputs by name, and the extent obligations fusion must not cross
    Store, ExtentWitness, NamedCast,
    // anything else the reader does not interpret
    Other
};
const char *op_name(Op op);
bool op_is_chain_step(Op op);  // fuse.rs's fusible elementwise table

// One step of a FusedElem: its op and its inputs, each an external input
// (>= 0) or a previous step k (encoded -(k + 1)), as FusedInput::External /
// FusedInput::PreviousStep.
struct Step {
    Op op = Op::Other;
    std::vector<int> args;
};

// An extent is a literal (>= 0) or the run-time extent of a symbol, coded
// as -2 - symbol. -1 marks an extent this build cannot bind (a bound read
// from a node value, or the to-the-end sentinel); Node::extent_error says
// which, and the planner refuses it.
constexpr int64_t kUnboundExtent = -1;
constexpr int64_t kToEnd = INT64_MIN;  // a shrink's to-the-end bound
inline bool extent_is_symbol(int64_t e) { return e <= -2; }
inline int64_t symbol_extent(int64_t symbol) { return -2 - symbol; }
inline int64_t extent_symbol(int64_t e) { return -2 - e; }

// The ExtentWitness sites whose owner no rewrite may merge away
// (crates/chelis-dag-core/src/axis_sources.rs:3736-3753).
enum class WitnessSite : uint8_t { None, LiteralResultClaim, ResultClaim, LocalAscriptionClaim, Other };

struct Node {
    int64_t id = 0;
    Op op = Op::Other;
    std::string variant;  // the op's variant name on the wire
    std::vector<int64_t> inputs, shape_deps, claim_deps;
    std::vector<int64_t> dims;  // extents (literal or symbol codes, above)
    std::vector<std::string> dims_raw;  // each DimInfo as read, written back verbatim
    std::string extent_error;           // why an extent is unbound, if one is
    Prim prec = Prim::Other;
    int64_t reusable = -1;
    bool has_span = false;
    std::string span;
    std::vector<std::string> merged_spans;
    int64_t owner_decl = 0, owner_activation = -1;
    // op fields
    int64_t axis = 0;               // Sum / MaxReduce / ... / Expand / Softmax
    std::vector<int64_t> axes;      // Permute / Count
    Prim accumulator = Prim::Other; // Sum
    int64_t size = -1;              // Expand (extent code)
    std::vector<int64_t> new_shape; // Reshape (extent codes)
    std::string name;               // Load / Store; ExtentWitness: the parameter it reads
    WitnessSite site = WitnessSite::None;  // ExtentWitness
    std::vector<int64_t> requirements;     // ExtentWitness: literal extents its axis must equal
    int64_t named_claims = 0;              // ExtentWitness: claims against other witnesses
    std::string compare;            // Compare / Logical kind (snake_case wire name)
    int64_t batch_rank = 0;         // Gather (its axis in `axis`)
    int32_t code = 0;               // ExtremaAdjoint: min (bit 0), right operand (bit 1); Split: the branch;
                                    // Cumsum: 1 for the decreasing direction (its axis in `axis`);
                                    // Bitwise: 0 and, 1 or, 2 xor, 3 shift left, 4 shift right
    // Pad: elements added before / after each axis (fill in const_*);
    // Shrink: start / end per axis (end kToEnd: the axis' end); Stride: the
    // step per axis. Extent codes as in dims.
    std::vector<int64_t> lo, hi, step;
    Prim const_prec = Prim::Other;  // Const
    uint64_t const_bits = 0;        // float bits, or the integer / bool value; ConstTensor: its element count
    std::vector<uint64_t> tensor_cells;  // ConstTensor: its elements' bytes, row-major, packed in 8-byte cells
    std::vector<Step> steps;        // FusedElem
    Prim cast_to = Prim::Other;     // Cast
    std::string raw_op;             // the op as read (written back verbatim)

    int64_t count() const;  // elements (-1 if any extent is not a literal)
    double const_value() const;
    // The inputs whose payload the op reads: an Expand or Reshape reads only
    // inputs[0] (later inputs are the tensors an InputAxis extent is read
    // from); a Store reads its one value.
    size_t payload_inputs() const { return (op == Op::Expand || op == Op::Reshape) ? 1 : inputs.size(); }
};

struct Graph {
    std::vector<Node> nodes;  // ids are positions, inputs precede users
    std::vector<int64_t> roots;
    std::string declarations = "[]";  // JSON text, carried through
    std::vector<std::string> symbols;  // run-time extent names, by symbol index

    int64_t symbol(const std::string &name);  // interned index
};

// Reads the reference's serde Dag; returns false with a message naming the
// offending node on any structural problem.
bool read_graph(const char *json, size_t n, Graph *g, std::string *error);
std::string write_graph(const Graph &g);

// ---------------------------------------------------------------- fusion
// fuse.rs:36-121: consumer counts (roots count as consumers), maximal chains
// of fusible float elementwise nodes where each link is its producer's only
// consumer and shares its owner, chains of length >= 2 rebuilt as FusedElem
// nodes; a node that owns a result claim (or a Copy / Cast / NamedCast
// such a node reads, transitively) neither starts nor joins a chain.
// old_to_new maps every old node to its node in the result.
Graph fuse(const Graph &g, std::vector<int64_t> *old_to_new);
// axis_sources.rs:3693-3753: the nodes whose shape or claim dependencies
// name a ResultClaim / LiteralResultClaim / LocalAscriptionClaim witness,
// closed over the first input of Copy, Cast and NamedCast.
std::vector<bool> claimed_producers(const Graph &g);
// fuse.rs:76-96 with the activation gate (dag.rs:2864-2880): whether the
// node may be a chain link at all.
bool chain_fusible(const Node &n);
// prepare_dag_for_codegen's BLAS selection (lib.rs:173-227, specialize.rs:
// 150-226): lowered matmuls as BlasMatmul nodes over strided operands (no
// Realize copies); idempotent.
Graph prepare_for_codegen(const Graph &g);
// fuse.rs:463-487: FusedElem nodes whose only consumer is a Sum or
// MaxReduce (they become that reduction's leaf).
std::vector<bool> reduction_inlined(const Graph &g);
// A FusedElem written back as its primitive nodes (inverse of fuse).
Graph unfuse(const Graph &g);
std::vector<int64_t> consumer_counts(const Graph &g);

// ---------------------------------------------------------------- plan
// A region is one launch. Its inputs are values (node ids); a value is
// either a caller input, a constant, a view of another value, or a
// materialized region output.
enum class RegionKind : uint8_t {
    Chain, Reduce, Count, Softmax, MaskedSoftmax, SoftmaxAdjoint, LayerNorm, Gelu, Relu, ReluAdjoint, Dropout,
    Matmul, Copy, Attention,
    // several products sharing their left operand, run as one batch
    MatmulGroup,
    // whole lowered programs recognized as one region (their results in
    // `out` and `more_out`): the linear-regression step and the MLP
    // training step, run as this library's fused programs
    LinregStep, MlpStep,
    // one node each: comparison, logical, where, checked cast, checked
    // integer arithmetic (code = the op), gather (axis, batch_rank)
    Compare, Logical, Where, Cast, Integer, Gather,
    // the extrema cotangent (code: min bit 0, right operand bit 1), a keyed
    // uniform draw
    ExtremaAdjoint, Uniform,
    // the ordered scan (axis, code: reverse); a pad (lo, fill); a scatter
    // (code: 0 replace, 1 add, 2 elements; axis, batch_rank)
    Scan, Pad, Scatter
};
const char *region_kind_name(RegionKind k);

struct Region {
    RegionKind kind = RegionKind::Chain;
    int64_t out = -1;                 // the node whose value the launch produces
    std::vector<int64_t> more_out;    // further results of a multi-result region
    std::vector<int64_t> in;          // value nodes read
    std::vector<int64_t> covers;      // every node the region computes
    chelis_fused_chain chain{};       // Chain / Reduce leaf
    bool has_chain = false;
    int32_t reduce_op = CHELIS_REDUCE_SUM;
    int64_t axis = 0;
    double scale = 1.0, epsilon = 0.0, rate = 0.0;
    int32_t causal = 0;
    bool replay = false;
    // matmul: in = {a, b[, bias][, residual]}
    bool has_bias = false, has_residual = false;
    int32_t activation = CHELIS_ACT_NONE;
    int32_t causal_mode = 0;  // 1: skip tiles above the diagonal, 2: clip the contraction
    // attention: in = {q [.., S, 64], k^T [.., 64, S], v [.., S, 64]}, scale
    // matmul group: in = {a, b_0, bias_0, b_1, bias_1, ...}, results out,
    // more_out in one workspace range, back to back
    // linreg step: in = {X, w, y}, out = grad, more_out = {loss}
    // mlp step: in = {x, onehot, w1, b1, w2, b2, key}, out = loss,
    // more_out = {w1', b1', w2', b2'}, rate, lr (below)
    double lr = 0.0;
    // compare / logical: the kind; integer: the CHELIS_INT_* op; gather's
    // batch rank (its axis in `axis`)
    int32_t code = 0;
    int64_t batch_rank = 0;
    // uniform_like: the bounds; uniform_like / dropout: a key derived while
    // planning (host_key), else the key is the last value in `in`
    double low = 0.0, high = 0.0;
    bool host_key = false;
    uint64_t key = 0;
    // pad: elements before each axis and the fill's bits
    std::vector<int64_t> lo;
    uint64_t fill = 0;
    std::vector<int64_t> outputs() const {
        std::vector<int64_t> o{out};
        o.insert(o.end(), more_out.begin(), more_out.end());
        return o;
    }
};

// How a value's storage is found at run time.
enum class Storage : uint8_t { Input, Const, View, Slot, Output, Inlined };
struct ValueInfo {
    Storage storage = Storage::Inlined;
    int64_t input = -1, output = -1;  // caller slot indices
    int64_t base = -1;                // View: the value it views
    int64_t slot = -1;                // Slot: workspace slot
    int64_t slot_offset = 0;          // Slot: bytes into the slot (a matmul group's later results)
    int64_t const_index = -1;         // Const: constant pool entry
    bool const_dense = false;         // a ConstTensor: row-major from const_index on
    // physical order of a materialized value: perm[i] = the logical axis
    // stored i-th (outermost first); empty = row-major
    std::vector<int64_t> layout;
};

// A workspace range: a literal byte count, or `coef` times the product of
// the run-time extents `symbols` (symbol indices, repeated for powers)
// rounded up to 256 bytes. Ranges are laid out back to back in slot order;
// with run-time extents the offsets are taken per run.
struct Slot {
    int64_t offset = 0, bytes = 0;  // literal slots
    int64_t coef = 0;               // run-time slots
    std::vector<int64_t> symbols;
    bool symbolic() const { return !symbols.empty(); }
};

// Where a run-time extent is read: the caller input slot and axis of the
// first Load declaring it (the reference's canonical binding source,
// emit.rs:1141-1150); every other Load axis naming it must agree.
struct SymbolRead {
    int64_t symbol = -1, input = -1, axis = -1;
};

// An ExtentWitness requirement checked before a run: the extent of the
// caller input's axis must equal `required` (spec/04 section 4.7 entry
// checks; a LiteralResultClaim witness checks nothing there, dag.rs:2582).
struct ExtentCheck {
    int64_t input = -1, axis = -1, required = 0;
    std::string parameter;
};

struct Plan {
    Graph graph;  // the unfused graph the regions refer to
    std::vector<Region> regions;
    std::vector<ValueInfo> values;  // per node
    std::vector<int64_t> input_nodes, output_nodes;
    std::vector<std::string> input_labels, output_labels;
    std::vector<Slot> slots;
    int64_t workspace_bytes = 0;       // -1 when a slot is sized at run time
    std::vector<uint64_t> const_bits;  // one element per constant, stored at its dtype width
    std::vector<Prim> const_prec;
    int64_t peak_device_bytes = 0;     // workspace + constants; -1 when sized at run time
    // run-time extents: symbolic_dims lists the graph's symbols in binding
    // order (their names); binds[k] reads symbolic_dims[k]; checks are the
    // other Load axes that must agree with a bound symbol
    std::vector<int64_t> symbolic_dims;
    std::vector<SymbolRead> binds, checks;
    std::vector<ExtentCheck> extent_checks;
};

bool build_plan(const Graph &input, Plan *plan, std::string *error);
std::string describe_plan(const Plan &plan);

// Run-time extents. values[s] is the extent of graph symbol s.
inline int64_t resolve_extent(int64_t e, const std::vector<int64_t> &values) {
    return extent_is_symbol(e) ? values[(size_t)extent_symbol(e)] : e;
}
std::vector<int64_t> resolve_dims(const std::vector<int64_t> &dims, const std::vector<int64_t> &values);
// Reads every symbol from the input shapes (rank-checked by the caller) and
// checks the agreeing axes; false with a message naming the input, axis
// and symbol on a mismatch or a negative extent.
bool bind_symbols(const Plan &plan, const int64_t *const *input_shapes, const int32_t *input_ranks,
                  std::vector<int64_t> *values, std::string *error);
// Lays the slots out for these extents: offsets[k], and the workspace size.
// False when a size overflows.
bool layout_slots(const Plan &plan, const std::vector<int64_t> &values, std::vector<int64_t> *offsets,
                  int64_t *workspace);
// The peak formula's text: one term per slot (a literal, or coef * names
// with a round_up(.., 256) where the coefficient is not a multiple of 256),
// then the constant pool; "0" when empty.
std::string peak_formula(const Plan &plan);

}  // namespace dag
}  // namespace chelis

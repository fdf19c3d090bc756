// The codegen surface (include/chelis_dag.h): what codegen_hip returns in
// the reference (HipCodegenResult, crates/chelis-backend-hip/src/lib.rs:
// 32-53,104-167), for this library. The generated host C++ embeds the DAG
// and defines the two generated entries with the reference's contracts and
// diagnostics:
//   {f}         host tensors in and out (emit.rs:667-808): count checks that
//               print "{f}: expected N inputs, got M" and abort, the input
//               shape preamble (emit.rs:1081-1200), inputs copied to fresh
//               device tensors, outputs from chelis_alloc under a write
//               lease, device synchronized before return;
//   {f}_device  device owners in, owned contiguous outputs
//               (emit.rs:838-964, spec/11-ffi.md:144-156): count checks,
//               null arrays trap "domain in entry", an input on another
//               device traps "domain in device_entry", then the device
//               shape preamble (emit.rs:1309-1395).
// Run-time extents are read from the inputs that declare them (the
// preamble's `chelis_device_metadata <name>` bindings) and size the outputs;
// the program is planned once per process, on first call.
#include <dlfcn.h>
#include <limits.h>
#include <stdlib.h>

#include <algorithm>
#include <string>
#include <vector>

#include "chelis_dag.h"
#include "dag.h"
#include "hip_common.h"

struct chelis_hip_codegen_result {
    std::string c_source, h_header, formula;
    std::vector<std::string> lists[5];  // compile, link, inputs, outputs, symbolic dims
    int64_t estimate = -1;
};

namespace chelis {
namespace dag {
namespace {

bool identifier(const std::string &s) {
    if (s.empty() || (s[0] >= '0' && s[0] <= '9')) return false;
    for (char c : s)
        if (!((c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') || c == '_')) return false;
    return true;
}

// The directory this library was loaded from, for the flags that find its
// headers (../include) and itself.
std::string library_dir() {
    Dl_info info{};
    if (!dladdr(reinterpret_cast<void *>(&chelis_codegen_hip), &info) || !info.dli_fname) return ".";
    std::string path = info.dli_fname;
    const size_t slash = path.rfind('/');
    return slash == std::string::npos ? "." : path.substr(0, slash);
}

std::string c_string_lines(const std::string &text) {
    std::string out;
    const size_t chunk = 96;
    for (size_t i = 0; i < text.size(); i += chunk) {
        out += "    " + json_quote(text.substr(i, chunk)) + "\n";
    }
    if (text.empty()) out = "    \"\"\n";
    return out;
}

// C source text of a string literal's contents, with '%' doubled so it can
// sit inside a printf format (the reference's sanitize_for_format_string).
std::string fmt_text(const std::string &s) {
    std::string q = json_quote(s);
    q = q.substr(1, q.size() - 2);
    std::string out;
    for (char c : q) {
        if (c == '%') out += "%%";
        else out += c;
    }
    return out;
}

const char *dtype_macro(Prim p) {
    switch (p) {
        case Prim::F32: return "CHELIS_DTYPE_F32";
        case Prim::F64: return "CHELIS_DTYPE_F64";
        case Prim::Int32: return "CHELIS_DTYPE_I32";
        case Prim::Bool: return "CHELIS_DTYPE_BOOL";
        case Prim::Int64: return "CHELIS_DTYPE_I64";
        case Prim::Bf16: return "CHELIS_DTYPE_BF16";
        case Prim::F16: return "CHELIS_DTYPE_F16";
        case Prim::Int8: return "CHELIS_DTYPE_I8";
        case Prim::Int16: return "CHELIS_DTYPE_I16";
        case Prim::Key: return "CHELIS_DTYPE_KEY";
        default: return "255";
    }
}

// The C variable a run-time extent is bound to: its own name when that is
// an identifier (as the reference emits it), else a numbered stand-in.
std::string symbol_var(const Graph &g, int64_t sym) {
    const std::string &name = g.symbols[(size_t)sym];
    return identifier(name) && name.rfind("chelis_", 0) != 0 ? name : "chelis_sym_" + std::to_string(sym);
}

struct Lines {
    std::string text;
    int indent = 1;
    void line(const std::string &l) { text += (l.empty() ? std::string() : std::string(4 * indent, ' ') + l) + "\n"; }
};

// The input shape preamble of either entry (emit.rs:1081-1200 host,
// :1309-1395 device): the host entry reads the runtime tensors, the device
// entry the owners' packets; then the symbol bindings, the witness
// requirements and the output shapes.
void shape_preamble(Lines &e, const Plan &plan, const std::string &f, bool device) {
    const Graph &g = plan.graph;
    std::vector<size_t> order(plan.input_labels.size());
    for (size_t k = 0; k < order.size(); ++k) order[k] = k;
    std::sort(order.begin(), order.end(),
              [&](size_t x, size_t y) { return plan.input_labels[x] < plan.input_labels[y]; });
    const std::string fn = fmt_text(f) + (device ? "_device" : "");
    for (size_t slot : order) {
        const Node &ld = g.nodes[plan.input_nodes[slot]];
        const std::string s = std::to_string(slot), label = fmt_text(plan.input_labels[slot]);
        e.line("if (inputs[" + s + "] == NULL) {");
        e.line("    fprintf(stderr, \"" + fn + ": input `" + label + "` at slot " + s + " is NULL\\n\");");
        e.line("    abort();");
        e.line("}");
        std::string dtype, rank, shape;
        if (device) {
            e.line("const chelis_gpu_tensor *input_view_" + s + " = chelis_device_tensor_view(inputs[" + s + "]);");
            dtype = "input_view_" + s + "->dtype";
            rank = "input_view_" + s + "->rank";
            shape = "input_view_" + s + "->shape[";
        } else {
            dtype = "chelis_tensor_read_view(inputs[" + s + "]).dtype";
            rank = "chelis_tensor_rank(inputs[" + s + "])";
            shape = "chelis_tensor_shape(inputs[" + s + "], ";
        }
        const std::string close = device ? "]" : ")";
        e.line("if (" + dtype + " != " + dtype_macro(ld.prec) +
               ") chelis_numeric_trap(\"numeric trap: domain in load at i64\");");
        const std::string r = std::to_string(ld.dims.size());
        e.line("if (" + rank + " != " + r + ") {");
        e.line("    fprintf(stderr, \"" + fn + ": input `" + label + "` expected rank " + r + ", got %d\\n\", " + rank +
               ");");
        e.line("    abort();");
        e.line("}");
        for (size_t a = 0; a < ld.dims.size(); ++a) {
            if (extent_is_symbol(ld.dims[a])) continue;
            const std::string ax = std::to_string(a), want = std::to_string(ld.dims[a]);
            e.line("if (" + shape + ax + close + " != " + want + ") {");
            e.line("    fprintf(stderr, \"" + fn + ": input `" + label + "` axis " + ax + " expected " + want +
                   ", got %lld\\n\", (long long)" + shape + ax + close + ");");
            e.line("    abort();");
            e.line("}");
        }
    }
    for (const SymbolRead &b : plan.binds) {
        const std::string var = symbol_var(g, b.symbol), name = fmt_text(g.symbols[(size_t)b.symbol]);
        auto read = [&](const SymbolRead &r) {
            return device ? "input_view_" + std::to_string(r.input) + "->shape[" + std::to_string(r.axis) + "]"
                          : "chelis_tensor_shape(inputs[" + std::to_string(r.input) + "], " + std::to_string(r.axis) +
                                ")";
        };
        e.line("chelis_device_metadata " + var + " = " + read(b) + ";");
        for (const SymbolRead &c : plan.checks) {
            if (c.symbol != b.symbol) continue;
            e.line("if (" + read(c) + " != " + var + ") {");
            e.line("    fprintf(stderr, \"" + fn + ": symbolic dim `" + name + "` mismatch: " +
                   fmt_text(plan.input_labels[c.input]) + "[" + std::to_string(c.axis) + "]=%lld but " + name +
                   "=%lld\\n\", (long long)" + read(c) + ", (long long)" + var + ");");
            e.line("    abort();");
            e.line("}");
        }
    }
    for (const ExtentCheck &c : plan.extent_checks) {
        const std::string rd = device ? "input_view_" + std::to_string(c.input) + "->shape[" + std::to_string(c.axis) + "]"
                                      : "chelis_tensor_shape(inputs[" + std::to_string(c.input) + "], " +
                                            std::to_string(c.axis) + ")";
        e.line("if (" + rd + " != " + std::to_string(c.required) + ") {");
        e.line("    fprintf(stderr, \"extent `" + fmt_text(c.parameter) + "`: claimed = %lld, " +
               fmt_text(c.parameter) + " axis " + std::to_string(c.axis) + " = %lld\\n\", (long long)" +
               std::to_string(c.required) + ", (long long)" + rd + ");");
        e.line("    chelis_numeric_trap(\"numeric trap: domain in load at i64\");");
        e.line("}");
    }
    // output shapes from the literal extents and the bound symbols
    for (size_t o = 0; o < plan.output_nodes.size(); ++o) {
        const Node &nd = g.nodes[plan.output_nodes[o]];
        std::string dims;
        for (size_t a = 0; a < nd.dims.size(); ++a)
            dims += (a ? ", " : "") +
                    (extent_is_symbol(nd.dims[a]) ? symbol_var(g, extent_symbol(nd.dims[a])) : std::to_string(nd.dims[a]));
        e.line("chelis_device_metadata chelis_output_shape_" + std::to_string(o) + "[" +
               std::to_string(std::max<size_t>(nd.dims.size(), 1)) + "] = { " + (dims.empty() ? "1" : dims) + " };");
    }
}

std::string emit_source(const Plan &plan, const Graph &fused, const std::string &f) {
    const Graph &g = plan.graph;
    std::string s;
    s += "// Generated by chelis_codegen_hip for `" + f + "` (gfx950): " + std::to_string(plan.regions.size()) +
         " launches; peak device bytes " + peak_formula(plan) + ".\n";
    s += "// Launch plan (index, region kind, result node, input nodes):\n";
    const std::string d = describe_plan(plan);
    size_t start = 0;
    while (start < d.size()) {
        const size_t end = d.find('\n', start);
        if (end == start) break;
        s += "//   " + d.substr(start, end - start) + "\n";
        if (end == std::string::npos) break;
        start = end + 1;
    }
    s += "#include <hip/hip_runtime_api.h>\n\n#include <cstdio>\n#include <cstdlib>\n#include <cstring>\n#include <mutex>\n\n"
         "#include \"chelis_dag.h\"\n#include \"chelis_device_owner.h\"\n#include \"chelis_hip.h\"\n"
         "#include \"chelis_runtime.h\"\n\n";
    s += "namespace {\n\n";
    s += "// the fused DAG this program was planned from (crates/chelis-dag-core wire form)\n";
    s += "const char kDag[] =\n" + c_string_lines(write_graph(fused)) + "    ;\n\n";
    const size_t n_in = plan.input_nodes.size(), n_out = plan.output_nodes.size();
    s += "const chelis_dtype kOutputDtypes[] = {";
    for (size_t o = 0; o < n_out; ++o) s += (o ? ", " : "") + std::string(dtype_macro(g.nodes[plan.output_nodes[o]].prec));
    if (!n_out) s += "0";
    s += "};\n\n";
    s += "chelis_dag_program *program() {\n"
         "    static std::once_flag once;\n    static chelis_dag_program *p = nullptr;\n"
         "    std::call_once(once, [] { p = chelis_dag_compile(kDag, (int64_t)(sizeof kDag - 1)); });\n"
         "    if (!p) {\n        fprintf(stderr, \"" + fmt_text(f) + ": %s\\n\", chelis_hip_last_error());\n"
         "        abort();\n    }\n    return p;\n}\n\n";
    s += "void hip_check(hipError_t e) {\n    if (e != hipSuccess) {\n"
         "        fprintf(stderr, \"HIP error: %s\\n\", hipGetErrorString(e));\n        abort();\n    }\n}\n\n";
    s += "chelis_device_tensor_owner *device_tensor(const chelis_device_metadata *shape, int32_t rank, "
         "chelis_dtype dtype) {\n"
         "    chelis_scalar dims[16];\n"
         "    for (int32_t a = 0; a < rank; ++a) dims[a] = chelis_scalar_from_bits(CHELIS_DTYPE_I64, (uint64_t)shape[a]);\n"
         "    chelis_scalar exemplar{};\n    exemplar.dtype = dtype;\n"
         "    return chelis_device_tensor_alloc(chelis_metadata_plan_new(\n"
         "        chelis_scalar_from_bits(CHELIS_DTYPE_I64, (uint64_t)rank), rank ? dims : nullptr, exemplar));\n}\n\n";
    // the run after the preamble: outputs allocated, the plan enqueued,
    // failures reported as the reference reports them
    auto run_tail = [&](Lines &e, bool device) {
        e.line("const chelis_gpu_tensor *chelis_in[" + std::to_string(std::max<size_t>(n_in, 1)) + "];");
        e.line("const chelis_gpu_tensor *chelis_out[" + std::to_string(std::max<size_t>(n_out, 1)) + "];");
        if (device) {
            for (size_t i = 0; i < n_in; ++i)
                e.line("chelis_in[" + std::to_string(i) + "] = input_view_" + std::to_string(i) + ";");
        } else {
            for (size_t i = 0; i < n_in; ++i) {
                const std::string k = std::to_string(i);
                e.line("chelis_device_metadata host_shape_" + k + "[16];");
                e.line("for (int32_t a = 0; a < chelis_tensor_rank(inputs[" + k + "]); ++a) host_shape_" + k +
                       "[a] = chelis_tensor_shape(inputs[" + k + "], a);");
                e.line("chelis_device_tensor_owner *din_" + k + " = device_tensor(host_shape_" + k +
                       ", chelis_tensor_rank(inputs[" + k + "]), chelis_tensor_read_view(inputs[" + k + "]).dtype);");
                e.line("chelis_device_tensor_copy_from_host(din_" + k + ", inputs[" + k + "]);");
                e.line("chelis_in[" + k + "] = chelis_device_tensor_view(din_" + k + ");");
            }
        }
        for (size_t o = 0; o < n_out; ++o) {
            const std::string k = std::to_string(o);
            const Node &nd = g.nodes[plan.output_nodes[o]];
            const std::string owner = device ? "outputs[" + k + "]" : "dout_" + k;
            e.line(std::string(device ? "" : "chelis_device_tensor_owner *") + owner + " = device_tensor(chelis_output_shape_" +
                   k + ", " + std::to_string(nd.dims.size()) + ", kOutputDtypes[" + k + "]);");
            e.line("chelis_out[" + k + "] = chelis_device_tensor_view(" + owner + ");");
        }
        e.line("const int32_t status = chelis_dag_run(program(), chelis_in, " + std::to_string(n_in) + ", chelis_out, " +
               std::to_string(n_out) + ");");
        // a launcher's own trap line (a gather's paired batch extents) is the
        // trap; any other domain error is the launch's
        e.line("if (status == CHELIS_HIP_EDOMAIN) {");
        e.line("    const char *why = chelis_hip_last_error();");
        e.line("    if (strncmp(why, \"numeric trap: \", 14) == 0) chelis_numeric_trap(why);");
        e.line("    fprintf(stderr, \"%s\\n\", why);");
        e.line("    chelis_numeric_trap(\"numeric trap: domain in launch at i64\");");
        e.line("}");
        e.line("if (status != CHELIS_HIP_OK) {");
        e.line("    fprintf(stderr, \"" + fmt_text(f) + ": %s\\n\", chelis_hip_last_error());");
        e.line("    abort();");
        e.line("}");
        bool traps = false;
        for (const Region &r : plan.regions)
            traps = traps || r.kind == RegionKind::Cast || r.kind == RegionKind::Integer ||
                    r.kind == RegionKind::Gather || r.kind == RegionKind::Scan ||
                    r.kind == RegionKind::Scatter;
        if (traps) {
            // the earliest failing launch's lowest failing element
            // ([04-NUM-15]), read once after the run
            e.line("{");
            e.line("    chelis_hip_numeric_failure chelis_failure;");
            e.line("    if (chelis_hip_take_numeric_failure(&chelis_failure) != CHELIS_HIP_OK) abort();");
            e.line("    if (chelis_failure.kind != 0) chelis_numeric_trap(chelis_failure.message);");
            e.line("}");
        }
        e.line("int32_t chelis_count_error = 0;");
        e.line("if (chelis_hip_trap_status(&chelis_count_error) != CHELIS_HIP_OK) abort();");
        e.line("if (chelis_count_error) {");
        e.line("    fprintf(stderr, \"numeric trap: domain in count at bool\");");
        e.line("    fprintf(stderr, \"\\n\");");
        e.line("    abort();");
        e.line("}");
        if (!device) {
            for (size_t o = 0; o < n_out; ++o) {
                const std::string k = std::to_string(o);
                const Node &nd = g.nodes[plan.output_nodes[o]];
                e.line("outputs[" + k + "] = chelis_alloc(" + std::to_string(nd.dims.size()) + ", chelis_output_shape_" +
                       k + ", kOutputDtypes[" + k + "]);");
                e.line("{");
                e.line("    chelis_tensor_write *lease = chelis_tensor_begin_write(outputs[" + k + "]);");
                e.line("    chelis_device_tensor_copy_to_host(lease, dout_" + k + ");");
                e.line("    chelis_tensor_end_write(lease);");
                e.line("}");
            }
        }
        e.line("hip_check(hipDeviceSynchronize());");
        if (!device) {
            for (size_t o = 0; o < n_out; ++o) e.line("chelis_device_tensor_release(dout_" + std::to_string(o) + ");");
            for (size_t i = 0; i < n_in; ++i) e.line("chelis_device_tensor_release(din_" + std::to_string(i) + ");");
        }
    };
    s += "}  // namespace\n\n";
    const std::string fn = fmt_text(f);
    // {f}_device
    {
        Lines e;
        e.line("if (n_in != " + std::to_string(n_in) + ") {");
        e.line("    fprintf(stderr, \"" + fn + "_device: expected %d inputs, got %d\\n\", " + std::to_string(n_in) +
               ", n_in);");
        e.line("    abort();");
        e.line("}");
        e.line("if (n_out != " + std::to_string(n_out) + ") {");
        e.line("    fprintf(stderr, \"" + fn + "_device: expected %d outputs, got %d\\n\", " + std::to_string(n_out) +
               ", n_out);");
        e.line("    abort();");
        e.line("}");
        e.line("");
        e.line("if ((n_in > 0 && inputs == NULL) || (n_out > 0 && outputs == NULL)) chelis_numeric_trap(\"numeric trap: "
               "domain in entry at i64\");");
        e.line("int current_device = 0;");
        e.line("hip_check(hipGetDevice(&current_device));");
        e.line("for (chelis_device_rank slot = 0; slot < n_in; ++slot) if (chelis_device_tensor_device(inputs[slot]) != "
               "current_device) chelis_numeric_trap(\"numeric trap: domain in device_entry at i64\");");
        shape_preamble(e, plan, f, true);
        e.line("");
        run_tail(e, true);
        s += "extern \"C\" void " + f + "_device(const chelis_device_tensor_owner *const *inputs, chelis_device_rank n_in, "
             "chelis_device_tensor_owner **outputs, chelis_device_rank n_out) {\n" + e.text + "}\n\n";
    }
    // {f}
    {
        Lines e;
        e.line("if (n_in != " + std::to_string(n_in) + ") {");
        e.line("    fprintf(stderr, \"" + fn + ": expected %d inputs, got %d\\n\", " + std::to_string(n_in) + ", n_in);");
        e.line("    abort();");
        e.line("}");
        e.line("if (n_out != " + std::to_string(n_out) + ") {");
        e.line("    fprintf(stderr, \"" + fn + ": expected %d outputs, got %d\\n\", " + std::to_string(n_out) +
               ", n_out);");
        e.line("    abort();");
        e.line("}");
        e.line("");
        e.line("if ((n_in > 0 && inputs == NULL) || (n_out > 0 && outputs == NULL)) chelis_numeric_trap(\"numeric trap: "
               "domain in entry at i64\");");
        shape_preamble(e, plan, f, false);
        e.line("");
        run_tail(e, false);
        s += "extern \"C\" void " + f + "(chelis_tensor **inputs, int n_in, chelis_tensor **outputs, int n_out) {\n" +
             e.text + "}\n";
    }
    return s;
}

}  // namespace
}  // namespace dag
}  // namespace chelis

using namespace chelis;
using namespace chelis::dag;

namespace {
thread_local std::string g_prepared;
}

extern "C" const char *chelis_prepare_dag_for_codegen(const char *json, int64_t length) {
    if (!json || length < 0) {
        set_error(CHELIS_HIP_EDOMAIN, "prepare_dag_for_codegen: null or negative-length text");
        return nullptr;
    }
    try {
        Graph g;
        std::string error;
        if (!read_graph(json, (size_t)length, &g, &error)) {
            set_error(CHELIS_HIP_EDOMAIN, "prepare_dag_for_codegen: %s", error.c_str());
            return nullptr;
        }
        g_prepared = write_graph(prepare_for_codegen(g));
        return g_prepared.c_str();
    } catch (const std::exception &e) {
        set_error(CHELIS_HIP_EHIP, "prepare_dag_for_codegen: %s", e.what());
        return nullptr;
    }
}

extern "C" int32_t chelis_hip_tensor_capable_prims(const chelis_dtype **prims) {
    // lib.rs:10-18, in its order: F32, F64, Bool, Bf16, F16, Int32, Int64
    static const chelis_dtype kPrims[] = {CHELIS_DTYPE_F32, CHELIS_DTYPE_F64, CHELIS_DTYPE_BOOL, CHELIS_DTYPE_BF16,
                                          CHELIS_DTYPE_F16, CHELIS_DTYPE_I32, CHELIS_DTYPE_I64};
    if (prims) *prims = kPrims;
    return (int32_t)(sizeof kPrims / sizeof kPrims[0]);
}

extern "C" const char *chelis_hip_runtime_dir(void) {
    static const std::string dir = [] {
        std::string d = library_dir() + "/../include";
        char buf[4096];
        if (realpath(d.c_str(), buf)) d = buf;
        return d;
    }();
    return dir.c_str();
}

extern "C" chelis_hip_codegen_result *chelis_codegen_hip(const char *json, int64_t length, const char *func_name) {
    if (!json || length < 0 || !func_name || !identifier(func_name)) {
        set_error(CHELIS_HIP_EDOMAIN, "codegen_hip: a DAG and a C identifier for the function name are required");
        return nullptr;
    }
    try {
        Graph g;
        std::string error;
        if (!read_graph(json, (size_t)length, &g, &error)) {
            set_error(CHELIS_HIP_EDOMAIN, "codegen_hip: %s", error.c_str());
            return nullptr;
        }
        const Graph fused = fuse(g, nullptr);
        Plan plan;
        if (!build_plan(fused, &plan, &error)) {
            set_error(CHELIS_HIP_EUNSUPPORTED, "codegen_hip: %s", error.c_str());
            return nullptr;
        }
        auto *r = new chelis_hip_codegen_result();
        const std::string f = func_name;
        r->c_source = emit_source(plan, fused, f);
        r->h_header = "#include \"chelis_device_owner.h\"\nextern \"C\" void " + f +
                      "(chelis_tensor **inputs, int n_in, chelis_tensor **outputs, int n_out);\nextern \"C\" void " +
                      f + "_device(const chelis_device_tensor_owner *const *inputs, chelis_device_rank n_in, "
                          "chelis_device_tensor_owner **outputs, chelis_device_rank n_out);";
        const std::string lib = library_dir();
        r->lists[0] = {"-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I" + lib + "/../include", "-I/opt/rocm/include"};
        r->lists[1] = {"-L" + lib, "-lchelis_hip", "-Wl,-rpath," + lib, "-L/opt/rocm/lib", "-lamdhip64"};
        r->lists[2] = plan.input_labels;
        r->lists[3] = plan.output_labels;
        for (int64_t sym : plan.symbolic_dims) r->lists[4].push_back(plan.graph.symbols[(size_t)sym]);
        r->formula = peak_formula(plan);
        r->estimate = plan.peak_device_bytes;
        return r;
    } catch (const std::exception &e) {
        set_error(CHELIS_HIP_EHIP, "codegen_hip: %s", e.what());
        return nullptr;
    }
}

extern "C" void chelis_codegen_release(chelis_hip_codegen_result *r) { delete r; }
extern "C" const char *chelis_codegen_c_source(const chelis_hip_codegen_result *r) { return r ? r->c_source.c_str() : ""; }
extern "C" const char *chelis_codegen_h_header(const chelis_hip_codegen_result *r) { return r ? r->h_header.c_str() : ""; }
extern "C" int32_t chelis_codegen_list_count(const chelis_hip_codegen_result *r, int32_t which) {
    return (r && which >= 0 && which < 5) ? (int32_t)r->lists[which].size() : -1;
}
extern "C" const char *chelis_codegen_list_item(const chelis_hip_codegen_result *r, int32_t which, int32_t index) {
    if (!r || which < 0 || which >= 5 || index < 0 || index >= (int32_t)r->lists[which].size()) return nullptr;
    return r->lists[which][index].c_str();
}
extern "C" const char *chelis_codegen_peak_device_bytes_formula(const chelis_hip_codegen_result *r) {
    return r ? r->formula.c_str() : "";
}
extern "C" int64_t chelis_codegen_peak_device_bytes_estimate(const chelis_hip_codegen_result *r) {
    return r ? r->estimate : -1;
}

struct chelis_hip_host_program_result {
    std::vector<std::string> names;
    std::vector<chelis_hip_codegen_result *> helpers;
    ~chelis_hip_host_program_result() {
        for (auto *h : helpers) delete h;
    }
};

extern "C" chelis_hip_host_program_result *chelis_codegen_hip_host_program(int32_t n_helpers,
                                                                           const char *const *names,
                                                                           const char *const *dags,
                                                                           const int64_t *lengths) {
    if (n_helpers < 0 || (n_helpers && (!names || !dags || !lengths))) {
        set_error(CHELIS_HIP_EDOMAIN, "codegen_hip_host_program: a helper manifest is required");
        return nullptr;
    }
    auto *r = new chelis_hip_host_program_result();
    try {
        for (int32_t h = 0; h < n_helpers; ++h) {
            Graph g;
            std::string error;
            if (!names[h] || !dags[h] || lengths[h] < 0 || !read_graph(dags[h], (size_t)lengths[h], &g, &error)) {
                set_error(CHELIS_HIP_EDOMAIN, "codegen_hip_host_program: helper %d: %s", h,
                          error.empty() ? "a name and a DAG are required" : error.c_str());
                delete r;
                return nullptr;
            }
            // lib.rs:245-256: the one selection predicate - a helper whose
            // DAG holds a Count runs on the device; there is no C fallback
            bool count = false;
            for (const Node &nd : g.nodes) count = count || nd.op == Op::Count;
            if (!count) continue;
            const std::string prepared = write_graph(prepare_for_codegen(g));
            chelis_hip_codegen_result *c =
                chelis_codegen_hip(prepared.c_str(), (int64_t)prepared.size(), names[h]);
            if (!c) {
                delete r;
                return nullptr;  // chelis_codegen_hip set the error, naming the helper's node
            }
            r->names.push_back(names[h]);
            r->helpers.push_back(c);
        }
        return r;
    } catch (const std::exception &e) {
        delete r;
        set_error(CHELIS_HIP_EHIP, "codegen_hip_host_program: %s", e.what());
        return nullptr;
    }
}

extern "C" void chelis_host_program_release(chelis_hip_host_program_result *r) { delete r; }
extern "C" int32_t chelis_host_program_helper_count(const chelis_hip_host_program_result *r) {
    return r ? (int32_t)r->helpers.size() : -1;
}
extern "C" const char *chelis_host_program_helper_name(const chelis_hip_host_program_result *r, int32_t i) {
    return (r && i >= 0 && i < (int32_t)r->names.size()) ? r->names[(size_t)i].c_str() : nullptr;
}
extern "C" const chelis_hip_codegen_result *chelis_host_program_helper(const chelis_hip_host_program_result *r,
                                                                       int32_t i) {
    return (r && i >= 0 && i < (int32_t)r->helpers.size()) ? r->helpers[(size_t)i] : nullptr;
}

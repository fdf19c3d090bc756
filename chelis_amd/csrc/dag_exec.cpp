// Running a planned DAG (include/chelis_dag.h): every value's packet is
// derived at run time (inputs are the caller's packets with their own
// strides; movement ops become views of them), intermediates are carved
// from one stream-ordered workspace, and each region is one call of this
// library's launchers on the library stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "chelis_dag.h"
#include "chelis_programs.h"
#include "dag.h"
#include "gemm.h"
#include "hip_common.h"

struct chelis_dag_program {
    chelis::dag::Plan plan;
    std::string description;
    std::mutex mutex;
    std::atomic<int32_t> mode{-1};  // chelis_dag_set_exact: -1 the library-wide mode at each run
    void *constants[64] = {};  // the constant pool on each device, uploaded on first use
    ~chelis_dag_program() {
        int here = -1;
        if (hipGetDevice(&here) != hipSuccess) return;
        for (int d = 0; d < 64; ++d) {
            if (!constants[d]) continue;
            if (hipSetDevice(d) == hipSuccess) (void)hipFree(constants[d]);
        }
        (void)hipSetDevice(here);
    }
};

namespace chelis {
namespace dag {
namespace {

struct Packet {
    std::vector<int64_t> shape, strides;
    chelis_gpu_tensor t{};
    bool live = false;
    void seal() {
        t.shape = shape.data();
        t.strides = strides.data();
        t.rank = (int32_t)shape.size();
        int64_t c = 1;
        for (int64_t e : shape) c *= e;
        t.count = c;
    }
};

int64_t span_elements(const Packet &p) {
    int64_t s = 0;
    for (size_t a = 0; a < p.shape.size(); ++a) {
        if (p.shape[a] == 0) return 0;
        s += (p.shape[a] - 1) * p.strides[a];
    }
    return s + 1;
}

// A view of `in` with `shape`, if one exists without moving data.
bool reshape_view(const Packet &in, const std::vector<int64_t> &shape, std::vector<int64_t> *strides) {
    strides->assign(shape.size(), 0);
    int64_t count = 1;
    for (int64_t e : shape) count *= e;
    if (count == 0 || count == 1) {
        int64_t acc = 1;
        for (size_t a = shape.size(); a-- > 0;) {
            (*strides)[a] = acc;
            acc *= std::max<int64_t>(shape[a], 1);
        }
        return true;
    }
    std::vector<int64_t> os, ost;
    for (size_t a = 0; a < in.shape.size(); ++a)
        if (in.shape[a] != 1) {
            os.push_back(in.shape[a]);
            ost.push_back(in.strides[a]);
        }
    size_t oi = 0, ni = 0;
    while (ni < shape.size() && oi < os.size()) {
        int64_t np = shape[ni], op = os[oi];
        size_t nj = ni + 1, oj = oi + 1;
        while (np != op) {
            if (np < op) {
                if (nj >= shape.size()) return false;
                np *= shape[nj++];
            } else {
                if (oj >= os.size()) return false;
                op *= os[oj++];
            }
        }
        for (size_t k = oi; k + 1 < oj; ++k)
            if (ost[k] != ost[k + 1] * os[k + 1]) return false;
        (*strides)[nj - 1] = ost[oj - 1];
        for (size_t k = nj - 1; k > ni; --k) (*strides)[k - 1] = (*strides)[k] * shape[k];
        ni = nj;
        oi = oj;
    }
    for (; ni < shape.size(); ++ni) (*strides)[ni] = 1;  // trailing extent-1 axes
    return oi == os.size();
}

bool rank_and_dtype_match(const Node &n, const chelis_gpu_tensor *t) {
    return t && t->rank == (int32_t)n.dims.size() && t->dtype == prim_dtype(n.prec);
}

bool type_matches(const Node &n, const chelis_gpu_tensor *t, const std::vector<int64_t> &values) {
    if (!rank_and_dtype_match(n, t)) return false;
    for (size_t a = 0; a < n.dims.size(); ++a)
        if (t->shape[a] != resolve_extent(n.dims[a], values)) return false;
    return true;
}

// Checks the inputs' ranks and dtypes and reads the run-time extents.
int32_t bind_inputs(const Plan &P, const chelis_gpu_tensor *const *inputs, int32_t n_in,
                    std::vector<int64_t> *values) {
    const Graph &g = P.graph;
    if (n_in != (int32_t)P.input_nodes.size())
        return set_error(CHELIS_HIP_EDOMAIN, "dag: expected %zu inputs, got %d", P.input_nodes.size(), n_in);
    if (n_in && !inputs) return set_error(CHELIS_HIP_EDOMAIN, "dag: null packet array");
    std::vector<const int64_t *> shapes((size_t)n_in);
    std::vector<int32_t> ranks((size_t)n_in);
    for (int32_t i = 0; i < n_in; ++i) {
        if (int32_t s = check_tensor(inputs[i], "dag input")) return s;
        if (!rank_and_dtype_match(g.nodes[P.input_nodes[i]], inputs[i]))
            return set_error(CHELIS_HIP_EDOMAIN, "dag: input %d (%s) does not have the program's rank and dtype", i,
                             P.input_labels[i].c_str());
        shapes[i] = inputs[i]->shape;
        ranks[i] = inputs[i]->rank;
    }
    std::string why;
    if (!bind_symbols(P, shapes.data(), ranks.data(), values, &why))
        return set_error(CHELIS_HIP_EDOMAIN, "dag: %s", why.c_str());
    for (int32_t i = 0; i < n_in; ++i)
        if (!type_matches(g.nodes[P.input_nodes[i]], inputs[i], *values))
            return set_error(CHELIS_HIP_EDOMAIN, "dag: input %d (%s) does not have the program's shape", i,
                             P.input_labels[i].c_str());
    for (const ExtentCheck &c : P.extent_checks) {
        const int64_t got = inputs[c.input]->shape[c.axis];
        if (got != c.required)
            return set_error(CHELIS_HIP_EDOMAIN, "dag: extent `%s` axis %lld: claimed = %lld, got %lld",
                             c.parameter.c_str(), (long long)c.axis, (long long)c.required, (long long)got);
    }
    return CHELIS_HIP_OK;
}

int32_t constant_pool(chelis_dag_program *prog, void **pool) {
    int device = 0;
    CHELIS_HIP_TRY(hipGetDevice(&device));
    if (device < 0 || device >= 64) return set_error(CHELIS_HIP_EHIP, "dag: device %d outside 0..63", device);
    std::lock_guard<std::mutex> lock(prog->mutex);
    const Plan &P = prog->plan;
    if (!prog->constants[device] && !P.const_bits.empty()) {
        std::vector<uint64_t> cells(P.const_bits.size());
        for (size_t k = 0; k < cells.size(); ++k) {
            const int64_t w = prim_width(P.const_prec[k]);
            uint64_t v = P.const_bits[k];
            cells[k] = w >= 8 ? v : (v & ((uint64_t(1) << (8 * w)) - 1));  // little-endian: low bytes first
        }
        void *p = nullptr;
        CHELIS_HIP_TRY(device_malloc(&p, cells.size() * 8));
        const hipError_t e = hipMemcpy(p, cells.data(), cells.size() * 8, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return set_error(CHELIS_HIP_EHIP, "dag: constant upload: %s", hipGetErrorString(e));
        }
        prog->constants[device] = p;
    }
    *pool = prog->constants[device];
    return CHELIS_HIP_OK;
}

const chelis_fused_chain &identity_chain() {
    // max_elem(a, a) selects a's stored bits (NaN payloads and -0 included)
    static const chelis_fused_chain c = [] {
        chelis_fused_chain x{};
        x.n_steps = 1;
        x.steps[0].op = CHELIS_FUSED_MAX_ELEM;
        return x;
    }();
    return c;
}

int32_t run_plan(chelis_dag_program *prog, const chelis_gpu_tensor *const *inputs, int32_t n_in,
                 const chelis_gpu_tensor *const *outputs, int32_t n_out) {
    const Plan &P = prog->plan;
    const Graph &g = P.graph;
    if (n_out != (int32_t)P.output_nodes.size())
        return set_error(CHELIS_HIP_EDOMAIN, "dag: expected %zu outputs, got %d", P.output_nodes.size(), n_out);
    if (n_out && !outputs) return set_error(CHELIS_HIP_EDOMAIN, "dag: null packet array");
    std::vector<int64_t> values;
    if (int32_t s = bind_inputs(P, inputs, n_in, &values)) return s;
    for (int32_t o = 0; o < n_out; ++o) {
        if (int32_t s = check_tensor(outputs[o], "dag output")) return s;
        if (!type_matches(g.nodes[P.output_nodes[o]], outputs[o], values))
            return set_error(CHELIS_HIP_EDOMAIN, "dag: output %d (%s) does not have the program's shape and dtype", o,
                             P.output_labels[o].c_str());
    }
    std::vector<int64_t> offsets;
    int64_t workspace = 0;
    if (!layout_slots(P, values, &offsets, &workspace))
        return set_error(CHELIS_HIP_EDOMAIN, "dag: the workspace for these extents overflows");
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    void *pool = nullptr;
    if (int32_t s = constant_pool(prog, &pool)) return s;
    char *ws = nullptr;
    if (workspace) {
        ws = static_cast<char *>(scratch_alloc((size_t)workspace));
        if (!ws) return set_error(CHELIS_HIP_EHIP, "dag: cannot allocate a %lld-byte workspace", (long long)workspace);
    }
    struct Release {
        char *p;
        size_t n;
        ~Release() { scratch_free(p, n); }
    } release{ws, (size_t)workspace};
    // ---- packets
    std::vector<Packet> pk(g.nodes.size());
    auto from = [](Packet &p, const chelis_gpu_tensor *t) {
        p.shape.assign(t->shape, t->shape + t->rank);
        p.strides.assign(t->strides, t->strides + t->rank);
        p.t = *t;
        p.t.ownership = 0;
        p.live = true;
        p.seal();
    };
    for (const Node &n : g.nodes) {
        const ValueInfo &v = P.values[n.id];
        Packet &p = pk[n.id];
        const std::vector<int64_t> dims = resolve_dims(n.dims, values);
        switch (v.storage) {
            case Storage::Input: from(p, inputs[v.input]); break;
            case Storage::Const:
                p.shape = dims;
                p.strides.assign(dims.size(), 0);
                p.t.data = static_cast<char *>(pool) + 8 * v.const_index;
                p.t.byte_capacity = 8;
                if (v.const_dense) {  // a literal tensor, row-major
                    int64_t acc = 1;
                    for (size_t a = dims.size(); a-- > 0;) {
                        p.strides[a] = acc;
                        acc *= std::max<int64_t>(dims[a], 1);
                    }
                    p.t.byte_capacity = 8 * (int64_t)((acc * prim_width(n.prec) + 7) / 8);
                }
                p.t.dtype = prim_dtype(n.prec);
                p.live = true;
                p.seal();
                break;
            case Storage::Slot: {
                p.shape = dims;
                p.strides.assign(dims.size(), 0);
                // dense in the stored order: layout[i] is the axis stored i-th
                int64_t acc = 1;
                if (v.layout.empty()) {
                    for (size_t a = dims.size(); a-- > 0;) {
                        p.strides[a] = acc;
                        acc *= std::max<int64_t>(dims[a], 1);
                    }
                } else {
                    for (size_t i = v.layout.size(); i-- > 0;) {
                        p.strides[v.layout[i]] = acc;
                        acc *= std::max<int64_t>(dims[v.layout[i]], 1);
                    }
                }
                const size_t k = (size_t)v.slot;
                p.t.data = ws + offsets[k] + v.slot_offset;
                p.t.byte_capacity = (k + 1 < offsets.size() ? offsets[k + 1] : workspace) - offsets[k] - v.slot_offset;
                p.t.dtype = prim_dtype(n.prec);
                p.live = true;
                p.seal();
                break;
            }
            case Storage::Output: {
                Packet out;
                from(out, outputs[v.output]);
                if (v.base == n.id) {
                    p = out;
                    p.seal();
                } else {
                    p.t = out.t;
                    p.shape = dims;
                    if (!reshape_view(out, dims, &p.strides))
                        return set_error(CHELIS_HIP_EUNSUPPORTED, "dag: output %lld is too strided to take node %lld",
                                         (long long)v.output, (long long)n.id);
                    p.live = true;
                    p.seal();
                }
                break;
            }
            case Storage::View: {
                const Packet &b = pk[v.base];
                if (!b.live) return set_error(CHELIS_HIP_EUNSUPPORTED, "dag: node %lld views a value with no storage",
                                              (long long)n.id);
                p.t = b.t;
                p.shape = dims;
                switch (n.op) {
                    case Op::Expand:
                        p.strides = b.strides;
                        p.strides.insert(p.strides.begin() + n.axis, 0);
                        break;
                    case Op::Permute:
                        p.strides.resize(n.axes.size());
                        for (size_t a = 0; a < n.axes.size(); ++a) p.strides[a] = b.strides[n.axes[a]];
                        break;
                    case Op::Reshape:
                        if (!reshape_view(b, dims, &p.strides))
                            return set_error(CHELIS_HIP_EUNSUPPORTED,
                                             "dag: node %lld reshapes a view that is not one run of memory",
                                             (long long)n.id);
                        break;
                    case Op::Shrink:
                    case Op::Stride: {
                        // element o of the view is element o * step + start of
                        // its operand; the bounds are checked against the
                        // operand's extents as they are at run time
                        const bool shrink = n.op == Op::Shrink;
                        int64_t offset = 0;
                        p.strides = b.strides;
                        for (size_t a = 0; a < dims.size(); ++a) {
                            const int64_t start = shrink ? n.lo[a] : 0, step = shrink ? 1 : n.step[a];
                            const int64_t end = shrink ? (n.hi[a] == kToEnd ? b.shape[a] : n.hi[a]) : 0;
                            const bool ok = shrink ? (start <= end && end <= b.shape[a] && dims[a] == end - start)
                                                   : (dims[a] == (b.shape[a] + step - 1) / step);
                            if (!ok)
                                return set_error(CHELIS_HIP_EDOMAIN,
                                                 "dag: node %lld: %s bounds do not fit its operand's extent %lld on "
                                                 "axis %zu",
                                                 (long long)n.id, shrink ? "shrink" : "stride",
                                                 (long long)b.shape[a], a);
                            if (dims[a] > 0) offset += start * b.strides[a];
                            p.strides[a] = b.strides[a] * step;
                        }
                        const int64_t bytes = offset * prim_width(n.prec);
                        p.t.data = static_cast<char *>(b.t.data) + bytes;
                        p.t.byte_capacity = b.t.byte_capacity - bytes;
                        break;
                    }
                    default:  // Realize / Copy / Store: the same bytes
                        p.strides = b.strides;
                        break;
                }
                p.live = true;
                p.seal();
                break;
            }
            default: break;
        }
        if (p.live && span_elements(p) * prim_width(n.prec) > p.t.byte_capacity && p.t.count)
            return set_error(CHELIS_HIP_EUNSUPPORTED, "dag: node %lld's view reaches past its storage", (long long)n.id);
    }
    // ---- launches
    for (const Region &r : P.regions) {
        std::vector<const chelis_gpu_tensor *> in;
        for (int64_t id : r.in) in.push_back(&pk[id].t);
        const chelis_gpu_tensor *out = &pk[r.out].t;
        int32_t s = CHELIS_HIP_OK;
        switch (r.kind) {
            case RegionKind::Chain:
                s = chelis_hip_fused_elementwise(&r.chain, in.data(), (int32_t)in.size(), out);
                break;
            case RegionKind::Reduce:
                s = chelis_hip_reduce(r.reduce_op, r.has_chain ? &r.chain : nullptr, in.data(), (int32_t)in.size(),
                                      (int32_t)r.axis, out);
                break;
            case RegionKind::Count:
                // a byte other than 0 / 1 goes to the trap channel, read once
                // by whoever waits for the run (chelis_hip_trap_status)
                s = chelis_hip_count(in[0], (int32_t)r.axis, out, nullptr);
                break;
            case RegionKind::Softmax: s = chelis_hip_softmax(in[0], out); break;
            case RegionKind::MaskedSoftmax:
                s = chelis_hip_scaled_masked_softmax(in[0], r.scale, r.causal, out);
                break;
            case RegionKind::SoftmaxAdjoint: s = chelis_hip_softmax_adjoint(in[0], in[1], out); break;
            case RegionKind::LayerNorm: s = chelis_hip_layer_norm(in[0], in[1], in[2], r.epsilon, out); break;
            case RegionKind::Gelu: s = chelis_hip_gelu(in[0], out); break;
            case RegionKind::Relu: s = chelis_hip_relu(in[0], out); break;
            case RegionKind::ReluAdjoint: s = chelis_hip_relu_adjoint(in[0], in[1], out); break;
            case RegionKind::Dropout:
                s = r.host_key ? (r.replay ? chelis_hip_dropout_replay(r.key, in[0], r.rate, out)
                                           : chelis_hip_dropout(r.key, in[0], r.rate, out))
                               : dropout_device_key(static_cast<const uint64_t *>(in[1]->data), in[0], r.rate, out);
                break;
            case RegionKind::Uniform:
                s = uniform_like_run(r.key, r.host_key ? nullptr : static_cast<const uint64_t *>(in[0]->data), r.low,
                                     r.high, out);
                break;
            case RegionKind::Pad: s = chelis_hip_pad(in[0], r.lo.data(), r.fill, out); break;
            case RegionKind::Scatter:
                s = r.code == 2 ? chelis_hip_scatter_elements(in[0], in[1], in[2], (int32_t)r.axis, out, nullptr)
                                : chelis_hip_scatter(r.code, in[0], in[1], in[2], (int32_t)r.axis,
                                                     (int32_t)r.batch_rank, out, nullptr);
                break;
            case RegionKind::Scan:
                s = chelis_hip_cumsum(in[0], (int32_t)r.axis, r.code, out, nullptr);
                break;
            case RegionKind::ExtremaAdjoint:
                s = chelis_hip_extrema_adjoint(r.code & 1, (r.code >> 1) & 1, in[0], in[1], in[2], out);
                break;
            case RegionKind::Matmul: {
                const chelis_gpu_tensor *bias = r.has_bias ? in[2] : nullptr;
                const chelis_gpu_tensor *res = r.has_residual ? in[r.has_bias ? 3 : 2] : nullptr;
                if (r.causal_mode && !bias && !res && r.activation == CHELIS_ACT_NONE)
                    s = matmul_causal(in[0], in[1], out, r.causal_mode);
                else if (bias || res || r.activation != CHELIS_ACT_NONE)
                    s = chelis_hip_linear(in[0], in[1], bias, r.activation, res, out, 0);
                else
                    s = chelis_hip_matmul(in[0], in[1], out, 0);
                break;
            }
            case RegionKind::Attention: {
                // k arrives as the k^T view the scores product read
                chelis_gpu_tensor kh = *in[1];
                int64_t shape[8], strides[8];
                for (int32_t a = 0; a < kh.rank; ++a) shape[a] = kh.shape[a], strides[a] = kh.strides[a];
                std::swap(shape[kh.rank - 1], shape[kh.rank - 2]);
                std::swap(strides[kh.rank - 1], strides[kh.rank - 2]);
                kh.shape = shape;
                kh.strides = strides;
                // collapse leading axes to [batch, heads] for the kernel's rank-4 form
                chelis_gpu_tensor t4[4];
                int64_t sh4[4][4], st4[4][4];
                const chelis_gpu_tensor *src[4] = {in[0], &kh, in[2], out};
                bool flat = true;
                for (int u = 0; u < 4; ++u) {
                    const chelis_gpu_tensor *t = src[u];
                    const int32_t rk = t->rank;
                    if (rk < 3 || rk > 4) { flat = false; break; }
                    t4[u] = *t;
                    if (rk == 3) {
                        sh4[u][0] = 1, st4[u][0] = t->shape[0] * t->strides[0];
                        for (int a = 0; a < 3; ++a) sh4[u][a + 1] = t->shape[a], st4[u][a + 1] = t->strides[a];
                    } else {
                        for (int a = 0; a < 4; ++a) sh4[u][a] = t->shape[a], st4[u][a] = t->strides[a];
                    }
                    t4[u].rank = 4;
                    t4[u].shape = sh4[u];
                    t4[u].strides = st4[u];
                }
                if (!flat || !attention_causal_fits(&t4[0], &t4[1], &t4[2], &t4[3])) {
                    s = set_error(CHELIS_HIP_EUNSUPPORTED,
                                  "dag: node %lld: attention operands are not [.., S, 64] views with a contiguous "
                                  "head axis", (long long)r.out);
                    break;
                }
                s = attention_causal(&t4[0], &t4[1], &t4[2], r.scale, &t4[3]);
                break;
            }
            // trapping launches record into the device's deferred failure
            // record, read once by whoever waits for the run
            // (chelis_hip_take_numeric_failure)
            case RegionKind::Compare: s = chelis_hip_compare(r.code, in[0], in[1], out); break;
            case RegionKind::Logical:
                s = chelis_hip_logical(r.code, in[0], in.size() > 1 ? in[1] : nullptr, out);
                break;
            case RegionKind::Where: s = chelis_hip_where(in[0], in[1], in[2], out); break;
            case RegionKind::Cast: s = chelis_hip_cast(in[0], out, nullptr); break;
            case RegionKind::Integer:
                s = chelis_hip_integer_elementwise(r.code, in[0], in.size() > 1 ? in[1] : nullptr, out, nullptr);
                break;
            case RegionKind::Gather:
                s = chelis_hip_gather(in[0], in[1], (int32_t)r.axis, (int32_t)r.batch_rank, out, nullptr);
                break;
            case RegionKind::Copy: {
                // floats through the identity chain (its vector paths);
                // other dtypes as raw elements (a pad with no padding)
                const chelis_gpu_tensor *dst = outputs[r.axis];
                if (dst->dtype == CHELIS_DTYPE_F32 || dst->dtype == CHELIS_DTYPE_F64) {
                    s = chelis_hip_fused_elementwise(&identity_chain(), in.data(), 1, dst);
                } else {
                    static const int64_t zeros[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                    s = chelis_hip_pad(in[0], zeros, 0, dst);
                }
                break;
            }
            case RegionKind::MatmulGroup: {
                // the results lie back to back in one range: one [n, M, N] block
                const int32_t nb = (int32_t)r.more_out.size() + 1;
                const chelis_gpu_tensor *w[8], *b[8];
                for (int32_t k = 0; k < nb; ++k) w[k] = in[1 + 2 * k], b[k] = in[2 + 2 * k];
                const int64_t M = out->shape[0], N = out->shape[1];
                const int64_t sh[3] = {nb, M, N}, stv[3] = {M * N, N, 1};
                chelis_gpu_tensor c3 = *out;
                c3.rank = 3, c3.shape = sh, c3.strides = stv, c3.count = nb * M * N;
                c3.byte_capacity = nb * M * N * dtype_width(out->dtype);
                s = linear_multi_b(in[0], w, b, nb, &c3);
                break;
            }
            case RegionKind::LinregStep: {
                const chelis_gpu_tensor *res[2] = {out, &pk[r.more_out[0]].t};
                s = chelis_prog_linreg_step(in.data(), 3, res, 2);
                break;
            }
            case RegionKind::MlpStep: {
                // the program writes dense results (as a chain region does)
                const std::vector<int64_t> outs = r.outputs();
                const chelis_gpu_tensor *res[5];
                for (size_t k = 0; k < outs.size(); ++k) {
                    res[k] = &pk[outs[k]].t;
                    if (!is_contiguous(res[k]) && !s)
                        s = set_error(CHELIS_HIP_EUNSUPPORTED, "dag: the MLP step writes dense results; node %lld is "
                                      "a strided view", (long long)outs[k]);
                }
                if (!s) s = mlp_train_step_run(in.data(), 7, res, 5, (float)r.rate, (float)r.lr);
                break;
            }
        }
        if (s) return s;
    }
    return CHELIS_HIP_OK;
}

}  // namespace
}  // namespace dag
}  // namespace chelis

using namespace chelis;
using namespace chelis::dag;

namespace {
thread_local std::string g_text;
}

extern "C" chelis_dag_program *chelis_dag_compile(const char *json, int64_t length) {
    if (!json || length < 0) {
        set_error(CHELIS_HIP_EDOMAIN, "dag: null or negative-length text");
        return nullptr;
    }
    try {
        Graph g;
        std::string error;
        if (!read_graph(json, (size_t)length, &g, &error)) {
            set_error(CHELIS_HIP_EDOMAIN, "dag: %s", error.c_str());
            return nullptr;
        }
        auto *prog = new chelis_dag_program();
        if (!build_plan(g, &prog->plan, &error)) {
            delete prog;
            set_error(CHELIS_HIP_EUNSUPPORTED, "dag: %s", error.c_str());
            return nullptr;
        }
        prog->description = describe_plan(prog->plan);
        return prog;
    } catch (const std::exception &e) {
        set_error(CHELIS_HIP_EHIP, "dag: %s", e.what());
        return nullptr;
    }
}

extern "C" void chelis_dag_release(chelis_dag_program *program) { delete program; }

extern "C" int32_t chelis_dag_run(chelis_dag_program *program, const chelis_gpu_tensor *const *inputs, int32_t n_in,
                                  const chelis_gpu_tensor *const *outputs, int32_t n_out) {
    if (!program) return set_error(CHELIS_HIP_EDOMAIN, "dag: null program");
    try {
        // one numeric mode for every launch of this run
        const ModeScope mode(program->mode.load(std::memory_order_relaxed));
        return run_plan(program, inputs, n_in, outputs, n_out);
    } catch (const std::exception &e) {
        return set_error(CHELIS_HIP_EHIP, "dag: %s", e.what());
    }
}

extern "C" int32_t chelis_dag_set_exact(chelis_dag_program *program, int32_t mode) {
    if (!program) return set_error(CHELIS_HIP_EDOMAIN, "dag: null program"), -2;
    return program->mode.exchange(mode < 0 ? -1 : (mode ? 1 : 0));
}

extern "C" int32_t chelis_dag_input_count(const chelis_dag_program *p) {
    return p ? (int32_t)p->plan.input_nodes.size() : -1;
}
extern "C" int32_t chelis_dag_output_count(const chelis_dag_program *p) {
    return p ? (int32_t)p->plan.output_nodes.size() : -1;
}

namespace {
const Node *slot_node(const chelis_dag_program *p, int32_t output, int32_t index) {
    if (!p) return nullptr;
    const auto &ids = output ? p->plan.output_nodes : p->plan.input_nodes;
    if (index < 0 || index >= (int32_t)ids.size()) return nullptr;
    return &p->plan.graph.nodes[ids[index]];
}
}  // namespace

extern "C" const char *chelis_dag_label(const chelis_dag_program *p, int32_t output, int32_t index) {
    if (!slot_node(p, output, index)) return nullptr;
    return (output ? p->plan.output_labels : p->plan.input_labels)[index].c_str();
}

extern "C" int32_t chelis_dag_type(const chelis_dag_program *p, int32_t output, int32_t index, int32_t *rank,
                                   int64_t *shape, int32_t shape_capacity, int32_t *dtype) {
    const Node *n = slot_node(p, output, index);
    if (!n) return set_error(CHELIS_HIP_EDOMAIN, "dag: no such slot");
    if (rank) *rank = (int32_t)n->dims.size();
    if (shape)
        for (int32_t a = 0; a < (int32_t)n->dims.size() && a < shape_capacity; ++a)
            shape[a] = extent_is_symbol(n->dims[a]) ? -1 : n->dims[a];
    if (dtype) *dtype = prim_dtype(n->prec);
    return CHELIS_HIP_OK;
}

extern "C" int64_t chelis_dag_peak_device_bytes(const chelis_dag_program *p) {
    return p ? p->plan.peak_device_bytes : -1;
}

extern "C" int32_t chelis_dag_symbol_count(const chelis_dag_program *p) {
    return p ? (int32_t)p->plan.symbolic_dims.size() : -1;
}

extern "C" const char *chelis_dag_symbol_name(const chelis_dag_program *p, int32_t index) {
    if (!p || index < 0 || index >= (int32_t)p->plan.symbolic_dims.size()) return nullptr;
    return p->plan.graph.symbols[(size_t)p->plan.symbolic_dims[(size_t)index]].c_str();
}

extern "C" int64_t chelis_dag_peak_device_bytes_at(const chelis_dag_program *p, const int64_t *values, int32_t n) {
    if (!p) return -1;
    const Plan &P = p->plan;
    if (n != (int32_t)P.symbolic_dims.size() || (n && !values)) {
        set_error(CHELIS_HIP_EDOMAIN, "dag: %zu run-time extents expected, got %d", P.symbolic_dims.size(), n);
        return -1;
    }
    std::vector<int64_t> v(P.graph.symbols.size(), 0);
    for (int32_t k = 0; k < n; ++k) {
        if (values[k] < 0) {
            set_error(CHELIS_HIP_EDOMAIN, "dag: a negative extent");
            return -1;
        }
        v[(size_t)P.symbolic_dims[(size_t)k]] = values[k];
    }
    std::vector<int64_t> offsets;
    int64_t ws = 0;
    if (!layout_slots(P, v, &offsets, &ws)) {
        set_error(CHELIS_HIP_EDOMAIN, "dag: the workspace for these extents overflows");
        return -1;
    }
    return ws + 8 * (int64_t)P.const_bits.size();
}

extern "C" int32_t chelis_dag_output_shape(const chelis_dag_program *p, const chelis_gpu_tensor *const *inputs,
                                           int32_t n_in, int32_t index, int32_t *rank, int64_t *shape,
                                           int32_t shape_capacity) {
    const Node *n = slot_node(p, 1, index);
    if (!n) return set_error(CHELIS_HIP_EDOMAIN, "dag: no such output");
    try {
        std::vector<int64_t> values;
        if (int32_t s = bind_inputs(p->plan, inputs, n_in, &values)) return s;
        if (rank) *rank = (int32_t)n->dims.size();
        if ((int32_t)n->dims.size() > shape_capacity && shape)
            return set_error(CHELIS_HIP_EDOMAIN, "dag: output rank %zu exceeds the capacity %d", n->dims.size(),
                             shape_capacity);
        if (shape)
            for (size_t a = 0; a < n->dims.size(); ++a) shape[a] = resolve_extent(n->dims[a], values);
        return CHELIS_HIP_OK;
    } catch (const std::exception &e) {
        return set_error(CHELIS_HIP_EHIP, "dag: %s", e.what());
    }
}

extern "C" int64_t chelis_dag_launch_count(const chelis_dag_program *p) {
    return p ? (int64_t)p->plan.regions.size() : -1;
}

extern "C" const char *chelis_dag_describe(const chelis_dag_program *p) { return p ? p->description.c_str() : ""; }

extern "C" const char *chelis_dag_fuse(const char *json, int64_t length) {
    if (!json || length < 0) {
        set_error(CHELIS_HIP_EDOMAIN, "dag: null or negative-length text");
        return nullptr;
    }
    Graph g;
    std::string error;
    if (!read_graph(json, (size_t)length, &g, &error)) {
        set_error(CHELIS_HIP_EDOMAIN, "dag: %s", error.c_str());
        return nullptr;
    }
    g_text = write_graph(fuse(g, nullptr));
    return g_text.c_str();
}

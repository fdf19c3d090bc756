// Region formation and memory planning for a lowered Chelis DAG.
//
// The reference's HIP emitter launches one kernel per fused node
// (crates/chelis-backend-hip/src/emit.rs:2472-3048) after fuse.rs's linear
// chains, so a softmax is four launches and a layer norm eight. Here the
// lowered forms the compiler writes are recognized whole and given to this
// library's region kernels:
//   matmul      Sum{L+1}(Mul(Expand{L+2}(a), Expand{L}(b))) (tier2.rs:706-857,
//               blas.rs:25-104) or BlasMatmul, with a following bias add,
//               relu or GELU graph and residual add folded into its epilogue
//   softmax     decompose_softmax (tier2.rs:1098-1178) over the last axis
//   masked      softmax(where(causal mask, s * scale, -inf)) (spec/05 4.7)
//   adjoint     y * (g - sum(g * y)) (grad.rs:2248)
//   layer norm  lower_layer_norm (tier2.rs:1248-1360)
//   gelu        activation.rs:145-149,183-276
// A pattern is taken only when every node it covers, other than its result,
// is read by nothing outside it (so nothing is computed twice); constants
// and inputs are shared freely. Everything else runs as fuse.rs would group
// it: maximal single-consumer chains of float elementwise ops (one
// FusedElem launch each), a chain or single elementwise node read only by a
// Sum / MaxReduce becomes that reduction's leaf (fuse.rs:463-487), and the
// remaining ops one launch each. Movement ops are views.
//
// The slot plan gives every materialized intermediate a 256-byte aligned
// range of one workspace, reusing a range once its last reader has been
// enqueued (the greedy non-overlapping reuse of spec/08-backends.md:285-297,
// crates/chelis-backend-hip/src/memory.rs:32-182).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <set>

#include "dag.h"

namespace chelis {
namespace dag {

// the most products one batched launch takes (the problem's per-batch
// weight and bias addresses, gemm.h kMaxBatchPtrs)
constexpr int kMaxGroup = 4;

const char *region_kind_name(RegionKind k) {
    switch (k) {
        case RegionKind::Chain: return "chain";
        case RegionKind::Reduce: return "reduce";
        case RegionKind::Count: return "count";
        case RegionKind::Softmax: return "softmax";
        case RegionKind::MaskedSoftmax: return "masked_softmax";
        case RegionKind::SoftmaxAdjoint: return "softmax_adjoint";
        case RegionKind::LayerNorm: return "layer_norm";
        case RegionKind::Gelu: return "gelu";
        case RegionKind::Relu: return "relu";
        case RegionKind::ReluAdjoint: return "relu_adjoint";
        case RegionKind::Dropout: return "dropout";
        case RegionKind::Matmul: return "matmul";
        case RegionKind::Copy: return "copy";
        case RegionKind::Attention: return "attention";
        case RegionKind::MatmulGroup: return "matmul_group";
        case RegionKind::LinregStep: return "linreg_step";
        case RegionKind::MlpStep: return "mlp_step";
        case RegionKind::Compare: return "compare";
        case RegionKind::Logical: return "logical";
        case RegionKind::Where: return "where";
        case RegionKind::Cast: return "cast";
        case RegionKind::Integer: return "integer";
        case RegionKind::Gather: return "gather";
        case RegionKind::ExtremaAdjoint: return "extrema_adjoint";
        case RegionKind::Uniform: return "uniform_like";
        case RegionKind::Scan: return "cumsum";
        case RegionKind::Pad: return "pad";
        case RegionKind::Scatter: return "scatter";
    }
    return "?";
}

namespace {

// ---------------------------------------------------------------- templates
// A template is a small graph in the shape a lowering writes, with numbered
// placeholders for the values it reads. match() maps it onto the DAG node
// for node (a template node may map to a node another template node also
// maps to, since the compiler may share equal constants).
struct TNode {
    Op op = Op::Other;
    int placeholder = -1;
    bool any_const = false;  // a Const of this type whatever its value
    std::vector<int> in;
    std::vector<int64_t> dims;
    Prim prec = Prim::Other;
    int64_t axis = 0, size = -1;
    std::vector<int64_t> axes;
    std::string compare;
    uint64_t bits = 0;
};

struct Template {
    std::vector<TNode> t;
    int add(TNode n) {
        t.push_back(std::move(n));
        return (int)t.size() - 1;
    }
    int ph(int k, std::vector<int64_t> dims, Prim p) {
        TNode n;
        n.placeholder = k;
        n.dims = std::move(dims);
        n.prec = p;
        return add(n);
    }
    int op(Op o, std::vector<int> in, std::vector<int64_t> dims, Prim p) {
        TNode n;
        n.op = o;
        n.in = std::move(in);
        n.dims = std::move(dims);
        n.prec = p;
        return add(n);
    }
    const TNode &at(int k) const { return t[k]; }
    int bin(Op o, int a, int b) { return op(o, {a, b}, t[a].dims, t[a].prec); }
    int un(Op o, int a) { return op(o, {a}, t[a].dims, t[a].prec); }
    int cnst(double v, std::vector<int64_t> dims, Prim p) {
        TNode n;
        n.op = Op::Const;
        n.dims = std::move(dims);
        n.prec = p;
        if (p == Prim::F32) {
            const float f = (float)v;
            uint32_t b;
            std::memcpy(&b, &f, 4);
            n.bits = b;
        } else if (p == Prim::F64) {
            std::memcpy(&n.bits, &v, 8);
        } else {
            n.bits = (uint64_t)(int64_t)v;
        }
        return add(n);
    }
    int any_const(std::vector<int64_t> dims, Prim p) {
        TNode n;
        n.op = Op::Const;
        n.any_const = true;
        n.dims = std::move(dims);
        n.prec = p;
        return add(n);
    }
    int expand(int x, int64_t axis, int64_t size) {
        std::vector<int64_t> d = t[x].dims;
        d.insert(d.begin() + axis, size);
        TNode n;
        n.op = Op::Expand;
        n.in = {x};
        n.dims = d;
        n.prec = t[x].prec;
        n.axis = axis;
        n.size = size;
        return add(n);
    }
    // tier2.rs:629-680: insert axes at 0 until the rank matches
    int expand_to(int x, const std::vector<int64_t> &target) {
        while (t[x].dims.size() < target.size()) {
            const size_t missing = target.size() - t[x].dims.size();
            x = expand(x, 0, target[missing - 1]);
        }
        return x;
    }
    int reduce(Op o, int x, int64_t axis) {
        std::vector<int64_t> d = t[x].dims;
        d.erase(d.begin() + axis);
        TNode n;
        n.op = o;
        n.in = {x};
        n.dims = d;
        n.prec = t[x].prec;
        n.axis = axis;
        return add(n);
    }
    int mean(int x, int64_t axis) {
        const int s = reduce(Op::Sum, x, axis);
        const int c = cnst((double)t[x].dims[axis], t[s].dims, t[x].prec);
        return bin(Op::Div, s, c);
    }
    int softmax(int x, int64_t axis) {
        const int64_t n = t[x].dims[axis];
        const int m = reduce(Op::MaxReduce, x, axis);
        const int e = un(Op::Exp, bin(Op::Sub, x, expand(m, axis, n)));
        const int s = reduce(Op::Sum, e, axis);
        return bin(Op::Div, e, expand(s, axis, n));
    }
    int permute(int x, std::vector<int64_t> axes) {
        std::vector<int64_t> d;
        for (int64_t a : axes) d.push_back(t[x].dims[a]);
        TNode n;
        n.op = Op::Permute;
        n.in = {x};
        n.dims = d;
        n.prec = t[x].prec;
        n.axes = std::move(axes);
        return add(n);
    }
    int reshape(int x, std::vector<int64_t> shape) { return op(Op::Reshape, {x}, std::move(shape), t[x].prec); }
    // a matmul in either form: BlasMatmul(a, b), or the lowered
    // Sum{L+1}(Mul(Expand{L+2}(a), Expand{L}(b))) (tier2.rs:706-857)
    int matmul(int a, int b) {
        std::vector<int64_t> d = t[a].dims;
        d.back() = t[b].dims.back();
        return op(Op::BlasMatmul, {a, b}, d, t[a].prec);
    }
    int linear(int x, int w, int b) {
        const int mm = matmul(x, w);
        return bin(Op::Add, mm, expand_to(b, t[mm].dims));
    }
};

struct Binding {
    std::vector<int64_t> map, ph;
    std::vector<int64_t> lowered;  // the Mul / Expand nodes of matched lowered matmuls
};

// The lowered matmul at graph node d: its operands, and the nodes between.
bool lowered_matmul(const Graph &g, int64_t d, int64_t *a, int64_t *b, int64_t inner[3]) {
    const Node &n = g.nodes[d];
    if (n.op != Op::Sum || n.inputs.size() != 1 || n.dims.size() < 2) return false;
    const Node &mul = g.nodes[n.inputs[0]];
    if (mul.op != Op::Mul || mul.inputs.size() != 2) return false;
    const Node &ea = g.nodes[mul.inputs[0]], &eb = g.nodes[mul.inputs[1]];
    const int64_t L = (int64_t)n.dims.size() - 2;
    if (ea.op != Op::Expand || eb.op != Op::Expand || n.axis != L + 1 || ea.axis != L + 2 || eb.axis != L)
        return false;
    const Node &A = g.nodes[ea.inputs[0]], &B = g.nodes[eb.inputs[0]];
    if (A.dims.size() != (size_t)L + 2 || B.dims.size() != (size_t)L + 2) return false;
    if (A.dims[L + 1] != B.dims[L] || ea.size != B.dims[L + 1] || eb.size != A.dims[L]) return false;
    *a = ea.inputs[0];
    *b = eb.inputs[0];
    inner[0] = n.inputs[0], inner[1] = mul.inputs[0], inner[2] = mul.inputs[1];
    return true;
}

bool match_node(const Template &T, int ti, const Graph &g, int64_t d, Binding &b) {
    if (b.map[ti] >= 0) return b.map[ti] == d;
    const TNode &t = T.at(ti);
    const Node &n = g.nodes[d];
    if (t.placeholder >= 0) {
        if (b.ph[t.placeholder] >= 0 && b.ph[t.placeholder] != d) return false;
        if (!t.dims.empty() && n.dims != t.dims) return false;
        if (t.prec != Prim::Other && n.prec != t.prec) return false;
        b.ph[t.placeholder] = d;
        b.map[ti] = d;
        return true;
    }
    if (t.op == Op::BlasMatmul && n.op == Op::Sum) {
        int64_t a, bb, inner[3];
        if (!lowered_matmul(g, d, &a, &bb, inner) || n.dims != t.dims || n.prec != t.prec) return false;
        b.map[ti] = d;
        b.lowered.insert(b.lowered.end(), inner, inner + 3);
        return match_node(T, t.in[0], g, a, b) && match_node(T, t.in[1], g, bb, b);
    }
    if (n.op != t.op || n.payload_inputs() != t.in.size() || n.dims != t.dims || n.prec != t.prec) return false;
    switch (t.op) {
        case Op::Sum: case Op::MaxReduce: if (n.axis != t.axis) return false; break;
        case Op::Expand: if (n.axis != t.axis || n.size != t.size) return false; break;
        case Op::Permute: if (n.axes != t.axes) return false; break;
        case Op::Compare: if (n.compare != t.compare) return false; break;
        case Op::Const: if (!t.any_const && (n.const_prec != t.prec || n.const_bits != t.bits)) return false; break;
        default: break;
    }
    b.map[ti] = d;
    for (size_t k = 0; k < t.in.size(); ++k)
        if (!match_node(T, t.in[k], g, n.inputs[k], b)) return false;
    return true;
}

bool match(const Template &T, int root, const Graph &g, int64_t d, int n_ph, Binding *b) {
    b->map.assign(T.t.size(), -1);
    b->ph.assign((size_t)n_ph, -1);
    b->lowered.clear();
    return match_node(T, root, g, d, *b);
}

// Several template roots onto several graph nodes under one binding.
bool match_all(const Template &T, const std::vector<int> &roots, const Graph &g, const std::vector<int64_t> &nodes,
               int n_ph, Binding *b) {
    b->map.assign(T.t.size(), -1);
    b->ph.assign((size_t)n_ph, -1);
    b->lowered.clear();
    if (roots.size() != nodes.size()) return false;
    for (size_t k = 0; k < roots.size(); ++k)
        if (!match_node(T, roots[k], g, nodes[k], *b)) return false;
    return true;
}

// ---------------------------------------------------------------- planner state
struct Planner {
    const Graph &g;
    std::vector<int64_t> counts;
    std::vector<std::vector<int64_t>> users;  // data consumers (inputs), each once, in node order
    std::vector<bool> is_root;
    std::vector<int> claimed;                 // region index, -1 free
    std::vector<bool> barrier;                // claimed producers (fuse.rs:147-161)
    std::vector<Region> regions;
    std::string error;

    explicit Planner(const Graph &graph, const std::vector<int64_t> &outputs) : g(graph) {
        counts = consumer_counts(g);
        users.resize(g.nodes.size());
        is_root.assign(g.nodes.size(), false);
        for (int64_t r : outputs) is_root[r] = true;
        // data readers only: the tensor an InputAxis extent is read from is
        // not read by the Expand / Reshape that names it
        for (const Node &n : g.nodes)
            for (size_t k = 0; k < n.payload_inputs(); ++k) {
                const int64_t i = n.inputs[k];
                if (users[i].empty() || users[i].back() != n.id) users[i].push_back(n.id);
            }
        claimed.assign(g.nodes.size(), -1);
        barrier = claimed_producers(g);
    }
    const Node &N(int64_t id) const { return g.nodes[id]; }
    bool free_leaf(int64_t id) const { return N(id).op == Op::Load || N(id).op == Op::Const; }

    // Every node of `cover` other than `out` and the free leaves is read
    // only inside `cover`, is no root, and is not yet in a region.
    bool closed(const std::set<int64_t> &cover, int64_t out) const {
        for (int64_t id : cover) {
            if (claimed[id] >= 0) return false;
            if (id == out || free_leaf(id)) continue;
            if (is_root[id]) return false;
            for (int64_t u : users[id])
                if (!cover.count(u)) return false;
        }
        return true;
    }
    static std::set<int64_t> image(const Binding &b, const Template &T) {
        std::set<int64_t> s(b.lowered.begin(), b.lowered.end());
        for (size_t k = 0; k < T.t.size(); ++k)
            if (T.t[k].placeholder < 0 && b.map[k] >= 0) s.insert(b.map[k]);
        return s;
    }
    // closed() for a region with several results
    bool closed_all(const std::set<int64_t> &cover, const std::vector<int64_t> &outs) const {
        for (int64_t id : cover) {
            if (claimed[id] >= 0 || barrier[id]) return false;
            const bool result = std::find(outs.begin(), outs.end(), id) != outs.end();
            if (result || free_leaf(id)) continue;
            if (is_root[id]) return false;
            for (int64_t u : users[id])
                if (!cover.count(u)) return false;
        }
        return true;
    }
    int claim(Region r) {
        const int idx = (int)regions.size();
        for (int64_t id : r.covers)
            if (!free_leaf(id)) claimed[id] = idx;
        for (int64_t o : r.outputs()) claimed[o] = idx;
        regions.push_back(std::move(r));
        return idx;
    }
    bool fail(const std::string &what) {
        if (error.empty()) error = what;
        return false;
    }
    // A Pad, Shrink or Stride this build cannot run: bounds read from node
    // values (RtDim::Node), a rank that differs from its operand's, or
    // literal bounds that do not produce the node's literal extents
    // (spec/05-risc-primitives.md section 2.4.1: a negative bound, a shrink
    // past its operand, a step below one).
    std::string window_error(const Node &n) const {
        if (n.inputs.size() != 1) return n.variant + " with bounds read from node values (run-time bounds)";
        const Node &src = N(n.inputs[0]);
        const size_t rk = src.dims.size();
        const std::vector<int64_t> &first = n.op == Op::Stride ? n.step : n.lo;
        if (first.size() != rk || n.dims.size() != rk) return n.variant + " bounds do not match its operand's rank";
        for (size_t a = 0; a < rk; ++a) {
            const int64_t f = first[a], h = n.op == Op::Stride ? 0 : n.hi[a];
            if (f < 0 || (h < 0 && !(n.op == Op::Shrink && h == kToEnd && f == 0)))
                return n.variant + " with a bound that is not a literal";
            if (n.op == Op::Stride && f < 1) return "Stride with a step below one";
            const int64_t se = src.dims[a], oe = n.dims[a];
            if (se < 0 || oe < 0) continue;  // run-time extents: checked when the program runs
            int64_t want = 0;
            if (n.op == Op::Pad) want = f + se + h;
            else if (n.op == Op::Stride) want = (se + f - 1) / f;
            else {
                const int64_t end = h == kToEnd ? se : h;
                if (end < f || end > se) return "Shrink bounds outside the operand on axis " + std::to_string(a);
                want = end - f;
            }
            if (want != oe) return n.variant + " bounds do not give the node's extent on axis " + std::to_string(a);
        }
        return "";
    }
    // The value of a Const, or of an Expand chain over one.
    bool const_of(int64_t id, double *v, Prim *p) const {
        while (N(id).op == Op::Expand || N(id).op == Op::Reshape) id = N(id).inputs[0];
        if (N(id).op != Op::Const) return false;
        *v = N(id).const_value();
        *p = N(id).const_prec;
        return true;
    }

    // ------------------------------------------------------------ patterns
    bool try_softmax(int64_t d) {
        const Node &n = N(d);
        if (n.op != Op::Div || n.dims.empty() || !prim_is_float(n.prec)) return false;
        const int64_t axis = (int64_t)n.dims.size() - 1;
        // softmax(where(causal mask, s * scale, -inf)) (spec/05 section 4.7 steps 3-5)
        const int64_t sq = n.dims.size() >= 2 ? n.dims[n.dims.size() - 2] : -1, sk = n.dims.back();
        for (const char *kind : {"gte", "lte"}) {
            if (sq != sk) break;
            Template T;
            const int s = T.ph(0, n.dims, n.prec);
            const int scale = T.expand_to(T.any_const({}, n.prec), n.dims);
            const int scaled = T.bin(Op::Mul, s, scale);
            const int ninf = T.expand_to(T.any_const({}, n.prec), n.dims);
            const int lo = T.any_const({}, Prim::Int64), hi = T.any_const({}, Prim::Int64);
            const int iota = T.op(Op::Iota, {lo, hi}, {sq}, Prim::Int64);
            const int rows = T.expand(iota, 1, sq), cols = T.expand(iota, 0, sq);
            TNode cmp;
            cmp.op = Op::Compare;
            cmp.compare = kind;
            cmp.in = std::string(kind) == "gte" ? std::vector<int>{rows, cols} : std::vector<int>{cols, rows};
            cmp.dims = {sq, sq};
            cmp.prec = Prim::Bool;
            const int mask = T.expand_to(T.add(cmp), n.dims);
            const int masked = T.op(Op::Where, {mask, scaled, ninf}, n.dims, n.prec);
            const int root = T.softmax(masked, axis);
            Binding b;
            if (!match(T, root, g, d, 1, &b)) continue;
            double sv, nv, lov, hiv;
            Prim sp, np_, lp, hp;
            if (!const_of(b.map[scale], &sv, &sp) || !const_of(b.map[ninf], &nv, &np_) ||
                !const_of(b.map[lo], &lov, &lp) || !const_of(b.map[hi], &hiv, &hp))
                continue;
            if (!(std::isinf(nv) && nv < 0) || lov != 0.0 || hiv != (double)sq) continue;
            std::set<int64_t> cover = image(b, T);
            if (!closed(cover, d)) continue;
            Region r;
            r.kind = RegionKind::MaskedSoftmax;
            r.out = d;
            r.in = {b.ph[0]};
            r.scale = sv;
            r.causal = 1;
            r.covers.assign(cover.begin(), cover.end());
            claim(r);
            return true;
        }
        // plain softmax over a placeholder
        {
            Template T;
            const int x = T.ph(0, n.dims, n.prec);
            const int root = T.softmax(x, axis);
            Binding b;
            if (match(T, root, g, d, 1, &b)) {
                std::set<int64_t> cover = image(b, T);
                if (closed(cover, d)) {
                    Region r;
                    r.kind = RegionKind::Softmax;
                    r.out = d;
                    r.in = {b.ph[0]};
                    r.covers.assign(cover.begin(), cover.end());
                    claim(r);
                    return true;
                }
            }
        }
        return false;
    }

    bool try_softmax_adjoint(int64_t d) {
        const Node &n = N(d);
        if (n.op != Op::Mul || n.dims.empty() || !prim_is_float(n.prec)) return false;
        const int64_t axis = (int64_t)n.dims.size() - 1;
        Template T;
        const int y = T.ph(0, n.dims, n.prec), gr = T.ph(1, n.dims, n.prec);
        const int s = T.reduce(Op::Sum, T.bin(Op::Mul, gr, y), axis);
        const int root = T.bin(Op::Mul, y, T.bin(Op::Sub, gr, T.expand(s, axis, n.dims[axis])));
        Binding b;
        if (!match(T, root, g, d, 2, &b)) return false;
        std::set<int64_t> cover = image(b, T);
        if (!closed(cover, d)) return false;
        Region r;
        r.kind = RegionKind::SoftmaxAdjoint;
        r.out = d;
        r.in = {b.ph[0], b.ph[1]};
        r.covers.assign(cover.begin(), cover.end());
        claim(r);
        return true;
    }

    bool try_layer_norm(int64_t d) {
        const Node &n = N(d);
        if (n.op != Op::Add || n.dims.empty() || !prim_is_float(n.prec)) return false;
        const std::vector<int64_t> &dims = n.dims;
        const int64_t axis = (int64_t)dims.size() - 1, h = dims[axis];
        Template T;
        const int x = T.ph(0, dims, n.prec), gamma = T.ph(1, {h}, n.prec), beta = T.ph(2, {h}, n.prec),
                  eps = T.ph(3, {}, n.prec);
        const int mean = T.mean(x, axis);
        const int centered = T.bin(Op::Sub, x, T.expand(mean, axis, h));
        const int var = T.mean(T.bin(Op::Mul, centered, centered), axis);
        const int denom = T.un(Op::Sqrt, T.bin(Op::Add, T.expand(var, axis, h), T.expand_to(eps, dims)));
        const int normed = T.bin(Op::Div, centered, denom);
        const int root =
            T.bin(Op::Add, T.bin(Op::Mul, normed, T.expand_to(gamma, dims)), T.expand_to(beta, dims));
        Binding b;
        if (!match(T, root, g, d, 4, &b)) return false;
        double ev;
        Prim ep;
        if (!const_of(b.ph[3], &ev, &ep)) return false;
        std::set<int64_t> cover = image(b, T);
        if (!closed(cover, d)) return false;
        Region r;
        r.kind = RegionKind::LayerNorm;
        r.out = d;
        r.in = {b.ph[0], b.ph[1], b.ph[2]};
        r.epsilon = ev;
        r.covers.assign(cover.begin(), cover.end());
        claim(r);
        return true;
    }

    // activation.rs:145-149,183-276 at the operand's dtype
    static int gelu_template(Template &T, const std::vector<int64_t> &dims, Prim p) {
        struct K {
            double c, cl, k, s, lowest;
        };
        const K k = p == Prim::F32
                        ? K{(double)(float)0.70710678118654752440, 1.2101617485882343e-8,
                            (double)(float)1.12837916709551257390, 4097.0, -3.4028234663852886e38}
                        : K{0.70710678118654752440, -4.833646656726457e-17, 1.12837916709551257390, 134217729.0,
                            -1.7976931348623157e308};
        const int x = T.ph(0, dims, p);
        const int lowest = T.cnst(k.lowest, dims, p);
        TNode below;
        below.op = Op::Compare;
        below.compare = "cmp_lt";
        below.in = {x, lowest};
        below.dims = dims;
        below.prec = Prim::Bool;
        const int bl = T.add(below);
        const int nzero = T.un(Op::Neg, T.cnst(0.0, dims, p));
        const int m = T.op(Op::Where, {bl, nzero, x}, dims, p);
        const int c = T.cnst(k.c, dims, p), cl = T.cnst(k.cl, dims, p), kk = T.cnst(k.k, dims, p),
                  s = T.cnst(k.s, dims, p);
        const int e = T.un(Op::Erfc, T.bin(Op::Mul, T.un(Op::Neg, x), c));
        TNode inside;
        inside.op = Op::Compare;
        inside.compare = "cmp_lt";
        inside.in = {T.un(Op::Abs, x), T.cnst(64.0, dims, p)};
        inside.dims = dims;
        inside.prec = Prim::Bool;
        const int in_ = T.add(inside);
        const int z = T.op(Op::Where, {in_, x, T.cnst(0.0, dims, p)}, dims, p);
        const int a = T.un(Op::Neg, z);
        const int th = T.bin(Op::Mul, a, c);
        const int ta = T.bin(Op::Mul, s, a);
        const int ah = T.bin(Op::Sub, ta, T.bin(Op::Sub, ta, a));
        const int al = T.bin(Op::Sub, a, ah);
        const int tc = T.bin(Op::Mul, s, c);
        const int ch = T.bin(Op::Sub, tc, T.bin(Op::Sub, tc, c));
        const int cr = T.bin(Op::Sub, c, ch);
        int err = T.bin(Op::Sub, T.bin(Op::Mul, ah, ch), th);
        err = T.bin(Op::Add, err, T.bin(Op::Mul, ah, cr));
        err = T.bin(Op::Add, err, T.bin(Op::Mul, al, ch));
        err = T.bin(Op::Add, err, T.bin(Op::Mul, al, cr));
        const int tl = T.bin(Op::Add, err, T.bin(Op::Mul, a, cl));
        const int dens = T.un(Op::Exp, T.un(Op::Neg, T.bin(Op::Mul, th, th)));
        const int corr = T.bin(Op::Mul, T.bin(Op::Mul, kk, dens), tl);
        const int phi = T.bin(Op::Mul, T.cnst(0.5, dims, p), T.bin(Op::Sub, e, corr));
        return T.bin(Op::Mul, m, phi);
    }

    // The GELU graph rooted at `d`; returns its input value or -1.
    int64_t gelu_at(int64_t d, std::set<int64_t> *cover) {
        const Node &n = N(d);
        if (n.op != Op::Mul || (n.prec != Prim::F32 && n.prec != Prim::F64)) return -1;
        Template T;
        const int root = gelu_template(T, n.dims, n.prec);
        Binding b;
        if (!match(T, root, g, d, 1, &b)) return -1;
        *cover = image(b, T);
        return b.ph[0];
    }

    bool try_gelu(int64_t d) {
        std::set<int64_t> cover;
        const int64_t x = gelu_at(d, &cover);
        if (x < 0 || !closed(cover, d)) return false;
        Region r;
        r.kind = RegionKind::Gelu;
        r.out = d;
        r.in = {x};
        r.covers.assign(cover.begin(), cover.end());
        claim(r);
        return true;
    }

    // ------------------------------------------------------------ whole programs
    // The linear-regression step as the compiler lowers it: r = X.w - y,
    // grad = X^T.r / n, loss = mean(r * r) (tier2.rs:706-857 for the
    // products, :1183-1245 for the mean), the roots [grad, loss]; run as
    // this library's linreg step (two launches where d <= 32), the same bits
    // as its unfused regions.
    bool try_linreg(const std::vector<int64_t> &outs) {
        if (outs.size() != 2) return false;
        const Node &grad = N(outs[0]), &loss = N(outs[1]);
        const Prim p = grad.prec;
        if ((p != Prim::F32 && p != Prim::F64) || grad.dims.size() != 1 || !loss.dims.empty() || loss.prec != p)
            return false;
        const int64_t d = grad.dims[0];
        for (const Node &ld : g.nodes) {
            if (ld.op != Op::Load || ld.dims.size() != 2 || ld.dims[1] != d || ld.prec != p) continue;
            const int64_t n = ld.dims[0];
            if (n < 0 || d < 0) continue;
            Template T;
            const int X = T.ph(0, {n, d}, p), w = T.ph(1, {d}, p), y = T.ph(2, {n}, p);
            const int r = T.bin(Op::Sub, T.reshape(T.matmul(X, T.reshape(w, {d, 1})), {n}), y);
            const int gs = T.matmul(T.permute(X, {1, 0}), T.reshape(r, {n, 1}));
            const int gt = T.bin(Op::Div, T.reshape(gs, {d}), T.cnst((double)n, {d}, p));
            const int lt = T.mean(T.bin(Op::Mul, r, r), 0);
            Binding b;
            if (!match_all(T, {gt, lt}, g, outs, 3, &b)) continue;
            std::set<int64_t> cover = image(b, T);
            if (!closed_all(cover, outs)) continue;
            Region rg;
            rg.kind = RegionKind::LinregStep;
            rg.out = outs[0];
            rg.more_out = {outs[1]};
            rg.in = {b.ph[0], b.ph[1], b.ph[2]};
            rg.covers.assign(cover.begin(), cover.end());
            claim(rg);
            return true;
        }
        return false;
    }

    // The MLP training step as the compiler lowers it (mnist.ch form):
    // forward relu(x.W1 + b1) -> dropout(key) -> softmax(. W2 + b2), loss
    // the mean cross-entropy against one-hot labels, its reverse pass
    // (mean, neg, sum, log and softmax adjoints, grad.rs:2248; transposed
    // products; dropout replay; relu adjoint) and SGD, the roots [loss, w1',
    // b1', w2', b2']; run as this library's MLP step (five launches where it
    // fits), the same bits as its unfused regions.
    bool try_mlp(const std::vector<int64_t> &outs) {
        if (outs.size() != 5) return false;
        const Node &w1n = N(outs[1]), &w2n = N(outs[3]);
        const Prim p = Prim::F32;
        if (w1n.prec != p || w1n.dims.size() != 2 || w2n.dims.size() != 2 || w2n.dims[0] != w1n.dims[1]) return false;
        const int64_t I = w1n.dims[0], Hd = w1n.dims[1], O = w2n.dims[1];
        for (const Node &ld : g.nodes) {
            if (ld.op != Op::Load || ld.dims.size() != 2 || ld.dims[1] != I || ld.prec != p || ld.dims[0] < 0) continue;
            const int64_t Bt = ld.dims[0];
            if (I < 0 || Hd < 0 || O < 0) continue;
            Template T;
            const int x = T.ph(0, {Bt, I}, p), oh = T.ph(1, {Bt, O}, p), w1 = T.ph(2, {I, Hd}, p),
                      b1 = T.ph(3, {Hd}, p), w2 = T.ph(4, {Hd, O}, p), b2 = T.ph(5, {O}, p),
                      key = T.ph(6, {}, Prim::Key);
            const int rate = T.any_const({}, p);
            const int z1 = T.linear(x, w1, b1);
            const int hd = T.un(Op::Relu, z1);
            const int d = T.op(Op::Dropout, {hd, rate, key}, {Bt, Hd}, p);
            const int pr = T.softmax(T.linear(d, w2, b2), 1);
            const int nl = T.un(Op::Neg, T.reduce(Op::Sum, T.bin(Op::Mul, T.un(Op::Log, pr), oh), 1));
            const int loss = T.mean(nl, 0);
            const int gsum = T.bin(Op::Div, T.cnst(1.0, {}, p), T.cnst((double)Bt, {}, p));
            const int gt = T.expand(T.un(Op::Neg, T.expand(gsum, 0, Bt)), 1, O);
            const int gp = T.bin(Op::Div, T.bin(Op::Mul, gt, oh), pr);
            const int gy = T.bin(Op::Mul, gp, pr);
            const int gz2 = T.bin(Op::Mul, pr, T.bin(Op::Sub, gp, T.expand(T.reduce(Op::Sum, gy, 1), 1, O)));
            const int gb2 = T.reduce(Op::Sum, gz2, 0);
            const int gw2 = T.matmul(T.permute(d, {1, 0}), gz2);
            const int gd = T.matmul(gz2, T.permute(w2, {1, 0}));
            const int gh = T.op(Op::DropoutReplay, {gd, rate, key}, {Bt, Hd}, p);
            const int gz1 = T.op(Op::ReluAdjoint, {z1, gh}, {Bt, Hd}, p);
            const int gb1 = T.reduce(Op::Sum, gz1, 0);
            const int gw1 = T.matmul(T.permute(x, {1, 0}), gz1);
            const int lr = T.any_const({}, p);
            auto sgd = [&](int w, int gw) {
                return T.bin(Op::Sub, w, T.bin(Op::Mul, T.expand_to(lr, T.at(w).dims), gw));
            };
            const std::vector<int> roots = {loss, sgd(w1, gw1), sgd(b1, gb1), sgd(w2, gw2), sgd(b2, gb2)};
            Binding b;
            if (!match_all(T, roots, g, outs, 7, &b)) continue;
            double rv, lv;
            Prim rp, lp;
            if (!const_of(b.map[rate], &rv, &rp) || !const_of(b.map[lr], &lv, &lp) || rp != p || lp != p) continue;
            if (!(rv >= 0.0 && rv < 1.0)) continue;
            std::set<int64_t> cover = image(b, T);
            if (!closed_all(cover, outs)) continue;
            Region rg;
            rg.kind = RegionKind::MlpStep;
            rg.out = outs[0];
            rg.more_out.assign(outs.begin() + 1, outs.end());
            rg.in.assign(b.ph.begin(), b.ph.end());
            rg.rate = rv;
            rg.lr = lv;
            rg.covers.assign(cover.begin(), cover.end());
            claim(rg);
            return true;
        }
        return false;
    }

    // matmul: Sum{L+1}(Mul(Expand{L+2, k}(a), Expand{L, i}(b))) or BlasMatmul
    bool try_matmul(int64_t d) {
        const Node &n = N(d);
        int64_t a = -1, b = -1;
        std::set<int64_t> cover{d};
        if (n.op == Op::BlasMatmul && n.inputs.size() == 2) {
            a = n.inputs[0];
            b = n.inputs[1];
        } else if (n.op == Op::Sum && n.inputs.size() == 1 && prim_is_float(n.prec)) {
            const Node &mul = N(n.inputs[0]);
            if (mul.op != Op::Mul || mul.inputs.size() != 2) return false;
            const Node &ea = N(mul.inputs[0]), &eb = N(mul.inputs[1]);
            if (ea.op != Op::Expand || eb.op != Op::Expand || ea.inputs.size() != 1 || eb.inputs.size() != 1)
                return false;
            const int64_t rank = (int64_t)mul.dims.size();  // [..., i, j, k]
            if (rank < 3) return false;
            const int64_t L = rank - 3;
            if (n.axis != L + 1 || ea.axis != L + 2 || eb.axis != L) return false;
            a = ea.inputs[0];
            b = eb.inputs[0];
            const Node &A = N(a), &B = N(b);
            if (A.dims.size() != (size_t)L + 2 || B.dims.size() != (size_t)L + 2) return false;
            if (A.dims[L + 1] != B.dims[L] || ea.size != B.dims[L + 1] || eb.size != A.dims[L]) return false;
            cover.insert({n.inputs[0], mul.inputs[0], mul.inputs[1]});
        } else {
            return false;
        }
        if (!closed(cover, d)) return false;
        Region r;
        r.kind = RegionKind::Matmul;
        r.in = {a, b};
        int64_t v = d;
        // epilogue: bias, then relu or GELU, then a residual add, each taken
        // only when it is the value's one reader
        auto sole_user = [&](int64_t id) -> int64_t {
            if (is_root[id] || users[id].size() != 1) return -1;
            return users[id][0];
        };
        int64_t bias = -1, residual = -1;
        int32_t act = CHELIS_ACT_NONE;
        int64_t u = sole_user(v);
        if (u >= 0 && N(u).op == Op::Add && N(u).inputs.size() == 2 && N(u).inputs[0] == v && claimed[u] < 0) {
            // the bias operand: expand_to_match of an [N] vector
            int64_t e = N(u).inputs[1];
            std::set<int64_t> chain{u};
            while (N(e).op == Op::Expand && N(e).axis == 0 && users[e].size() == 1 && !is_root[e]) {
                chain.insert(e);
                e = N(e).inputs[0];
            }
            if (N(e).dims.size() == 1 && N(e).dims[0] == N(v).dims.back() && N(e).prec == N(v).prec &&
                chain.size() == N(v).dims.size()) {
                bias = e;
                cover.insert(chain.begin(), chain.end());
                v = u;
            }
        }
        u = sole_user(v);
        if (u >= 0 && N(u).op == Op::Relu && claimed[u] < 0) {
            act = CHELIS_ACT_RELU;
            cover.insert(u);
            v = u;
        } else if (!is_root[v]) {
            // the GELU graph reads its input at several nodes; its result is
            // the Mul of the guard's Where
            for (int64_t w : users[v]) {
                if (N(w).op != Op::Where || N(w).inputs.size() != 3 || N(w).inputs[2] != v) continue;
                for (int64_t f : users[w]) {
                    std::set<int64_t> gc;
                    if (gelu_at(f, &gc) != v) continue;
                    std::set<int64_t> all = cover;
                    all.insert(gc.begin(), gc.end());
                    all.insert(v);
                    if (!closed(all, f)) continue;
                    cover = all;
                    act = CHELIS_ACT_GELU;
                    v = f;
                    break;
                }
                if (act == CHELIS_ACT_GELU) break;
            }
        }
        u = sole_user(v);
        if (u >= 0 && N(u).op == Op::Add && N(u).inputs.size() == 2 && claimed[u] < 0) {
            const int64_t other = N(u).inputs[0] == v ? N(u).inputs[1] : N(u).inputs[0];
            if (other != v && N(other).dims == N(v).dims && N(other).prec == N(v).prec) {
                residual = other;
                cover.insert(u);
                v = u;
            }
        }
        r.out = v;
        if (bias >= 0) {
            r.in.push_back(bias);
            r.has_bias = true;
        }
        if (residual >= 0) {
            r.in.push_back(residual);
            r.has_residual = true;
        }
        r.activation = act;
        cover.insert(v);
        r.covers.assign(cover.begin(), cover.end());
        claim(r);
        return true;
    }

    // ------------------------------------------------------------ generic regions
    static int chain_op(Op op) {
        switch (op) {
            case Op::Add: return CHELIS_FUSED_ADD;
            case Op::Sub: return CHELIS_FUSED_SUB;
            case Op::Mul: return CHELIS_FUSED_MUL;
            case Op::Div: return CHELIS_FUSED_DIV;
            case Op::MaxElem: return CHELIS_FUSED_MAX_ELEM;
            case Op::MinElem: return CHELIS_FUSED_MIN_ELEM;
            case Op::Neg: return CHELIS_FUSED_NEG;
            case Op::Recip: return CHELIS_FUSED_RECIP;
            case Op::Exp: return CHELIS_FUSED_EXP;
            case Op::Log: return CHELIS_FUSED_LOG;
            case Op::Sqrt: return CHELIS_FUSED_SQRT;
            case Op::Tanh: return CHELIS_FUSED_TANH;
            case Op::Erfc: return CHELIS_FUSED_ERFC;
            case Op::Abs: return CHELIS_FUSED_ABS;
            case Op::Floor: return CHELIS_FUSED_FLOOR;
            case Op::Ceil: return CHELIS_FUSED_CEIL;
            case Op::Round: return CHELIS_FUSED_ROUND;
            default: return -1;
        }
    }
    bool fusible(int64_t id) const {
        const Node &n = N(id);
        return claimed[id] < 0 && op_is_chain_step(n.op) && prim_is_float(n.prec) && chain_fusible(n) &&
               !barrier[id];
    }

    // Build chelis_fused_chain launches from a run of chain nodes; nodes
    // beyond 16 steps or 8 external inputs start a new launch whose result
    // feeds the next. Returns the regions' indices.
    bool emit_chain(const std::vector<int64_t> &nodes, int64_t reduce_node) {
        size_t start = 0;
        while (start < nodes.size()) {
            Region r;
            r.kind = RegionKind::Chain;
            r.has_chain = true;
            std::vector<int64_t> ext;
            std::vector<int64_t> steps;
            size_t k = start;
            for (; k < nodes.size(); ++k) {
                const Node &n = N(nodes[k]);
                std::vector<int64_t> need;
                for (int64_t in : n.inputs)
                    if (std::find(steps.begin(), steps.end(), in) == steps.end() &&
                        std::find(ext.begin(), ext.end(), in) == ext.end() &&
                        std::find(need.begin(), need.end(), in) == need.end())
                        need.push_back(in);
                if (steps.size() + 1 > CHELIS_FUSED_MAX_STEPS || ext.size() + need.size() > CHELIS_FUSED_MAX_INPUTS)
                    break;
                const int cop = chain_op(n.op);
                if (cop < 0) return fail(std::string("node ") + std::to_string(n.id) + ": " + op_name(n.op) +
                                         " has no device chain step in this build");
                ext.insert(ext.end(), need.begin(), need.end());
                chelis_fused_step &s = r.chain.steps[steps.size()];
                s.op = (uint8_t)cop;
                for (size_t a = 0; a < 2; ++a) {
                    const int64_t in = n.inputs[a < n.inputs.size() ? a : 0];
                    auto sp = std::find(steps.begin(), steps.end(), in);
                    s.args[a] = sp != steps.end() ? -(int32_t)(sp - steps.begin()) - 1
                                                  : (int32_t)(std::find(ext.begin(), ext.end(), in) - ext.begin());
                }
                steps.push_back(n.id);
            }
            if (k == start) return fail("a chain step needs more than 8 inputs");
            r.chain.n_steps = (int32_t)steps.size();
            r.in = ext;
            r.covers = steps;
            r.out = steps.back();
            const bool last = k == nodes.size();
            if (last && reduce_node >= 0) {
                const Node &red = N(reduce_node);
                r.kind = RegionKind::Reduce;
                r.reduce_op = red.op == Op::Sum ? CHELIS_REDUCE_SUM : CHELIS_REDUCE_MAX;
                r.axis = red.axis;
                r.covers.push_back(reduce_node);
                r.out = reduce_node;
            }
            claim(r);
            start = k;
        }
        return true;
    }

    // fuse.rs would join an integer node and its one reader into a FusedElem
    // chain (its fusibility table holds integer add, mul, neg, floor_div and
    // trunc_div); both reference lanes refuse integer chains.
    bool int_fusible(int64_t id) const {
        const Node &n = N(id);
        return claimed[id] < 0 && op_is_chain_step(n.op) && is_integer(n.prec) && chain_fusible(n) && !barrier[id];
    }
    bool in_integer_chain(int64_t id) const {
        if (!int_fusible(id)) return false;
        auto link = [&](int64_t p) {
            if (counts[p] != 1 || users[p].size() != 1) return false;
            const int64_t c = users[p][0];
            return int_fusible(p) && int_fusible(c) && N(c).owner_decl == N(p).owner_decl &&
                   N(c).owner_activation == N(p).owner_activation;
        };
        if (link(id)) return true;
        for (int64_t in : N(id).inputs)
            if (link(in) && users[in][0] == id) return true;
        return false;
    }
    static int int_code(Op op) {
        switch (op) {
            case Op::Add: return CHELIS_INT_ADD;
            case Op::Sub: return CHELIS_INT_SUB;
            case Op::Mul: return CHELIS_INT_MUL;
            case Op::FloorDiv: return CHELIS_INT_FLOOR_DIV;
            case Op::TruncDiv: return CHELIS_INT_TRUNC_DIV;
            case Op::Mod: return CHELIS_INT_MOD;
            case Op::MaxElem: return CHELIS_INT_MAX_ELEM;
            case Op::MinElem: return CHELIS_INT_MIN_ELEM;
            case Op::Neg: return CHELIS_INT_NEG;
            case Op::Abs: return CHELIS_INT_ABS;
            default: return -1;
        }
    }
    // [05-RNG-1/2] on the host: splitmix64, derive(k, j) =
    // splitmix64(k ^ rotl64(splitmix64(j), 29)) (dtype_semantics.rs:4039-4060)
    static uint64_t splitmix(uint64_t x) {
        x += 0x9e3779b97f4a7c15ull;
        x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
        x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
        return x ^ (x >> 31);
    }
    static uint64_t derive(uint64_t k, uint64_t j) {
        const uint64_t e = splitmix(j);
        return splitmix(k ^ ((e << 29) | (e >> 35)));
    }
    // The key a rank-0 key node holds when it is derived from literal seeds
    // and indices alone, as the reference derives draw keys at emission
    // (emit.rs:3594-3653): key_from_seed is the seed's bits, split a derive
    // by the branch, fold_in derive(derive(k, 2), n).
    bool derived_key(int64_t id, uint64_t *k) const {
        const Node &n = N(id);
        if (!n.dims.empty() || n.prec != Prim::Key) return false;
        double v;
        Prim p;
        switch (n.op) {
            case Op::KeyFromSeed:
                if (n.inputs.size() != 1 || N(n.inputs[0]).op != Op::Const || N(n.inputs[0]).const_prec != Prim::Int64)
                    return false;
                *k = N(n.inputs[0]).const_bits;
                return true;
            case Op::SplitKey:
                if (n.inputs.size() != 1 || !derived_key(n.inputs[0], k)) return false;
                *k = derive(*k, (uint64_t)n.code);
                return true;
            case Op::FoldIn:
                if (n.inputs.size() != 2 || !derived_key(n.inputs[0], k) || !const_of(n.inputs[1], &v, &p) ||
                    p != Prim::Int64 || N(n.inputs[1]).op != Op::Const)
                    return false;
                *k = derive(derive(*k, 2), N(n.inputs[1]).const_bits);
                return true;
            default:
                return false;
        }
    }
    static int compare_code(const std::string &k) {
        static const char *names[] = {"cmp_lt", "lt", "eq", "neq", "gt", "gte", "lte"};
        for (int i = 0; i < 7; ++i)
            if (k == names[i]) return i;
        return -1;
    }
    bool single(const Node &n, RegionKind kind, int32_t code = 0) {
        Region r;
        r.kind = kind;
        r.code = code;
        r.in = n.inputs;
        r.out = n.id;
        r.covers = {n.id};
        claim(r);
        return true;
    }

    bool generic() {
        for (const Node &n : g.nodes) {
            if (claimed[n.id] >= 0) continue;
            if (is_integer(n.prec) && in_integer_chain(n.id))
                return fail("node " + std::to_string(n.id) + ": " + n.variant +
                            " would join an integer fused elementwise chain, which neither reference lane runs "
                            "(crates/chelis-backend-c/src/emit.rs:6933-6945)");
            if (is_integer(n.prec) && int_code(n.op) >= 0 && n.owner_activation < 0) {
                const size_t want = (n.op == Op::Neg || n.op == Op::Abs) ? 1 : 2;
                if (n.inputs.size() != want)
                    return fail("node " + std::to_string(n.id) + ": " + n.variant + " with the wrong arity");
                single(n, RegionKind::Integer, int_code(n.op));
                continue;
            }
            if (fusible(n.id)) {
                // fuse.rs:136-191: extend through single-consumer fusible links
                std::vector<int64_t> chain{n.id};
                int64_t cur = n.id;
                while (counts[cur] == 1 && users[cur].size() == 1) {
                    const int64_t c = users[cur][0];
                    if (!fusible(c) || N(c).owner_decl != n.owner_decl ||
                        N(c).owner_activation != n.owner_activation ||
                        std::find(chain.begin(), chain.end(), c) != chain.end())
                        break;
                    chain.push_back(c);
                    cur = c;
                }
                // a chain whose one reader is a Sum or MaxReduce is its leaf
                int64_t red = -1;
                if (counts[cur] == 1 && users[cur].size() == 1) {
                    const int64_t c = users[cur][0];
                    if (claimed[c] < 0 && (N(c).op == Op::Sum || N(c).op == Op::MaxReduce) && N(c).inputs[0] == cur)
                        red = c;
                }
                if (!emit_chain(chain, red)) return false;
                continue;
            }
            switch (n.op) {
                case Op::Load: case Op::Const: case Op::Expand: case Op::Permute: case Op::Reshape:
                case Op::Realize: case Op::Copy: case Op::Store: case Op::Drop:
                    continue;  // inputs, constants, views and releases
                case Op::ConstTensor: {
                    const int64_t c = n.count();
                    if (c < 0 || (uint64_t)c != n.const_bits || n.const_prec != n.prec)
                        return fail("node " + std::to_string(n.id) +
                                    ": ConstTensor data does not fill the node's literal extents at its dtype");
                    continue;
                }
                case Op::Shrink: case Op::Stride: {
                    // views of their operand (an offset, scaled strides),
                    // as the reference HIP lane's stride is (emit.rs:4918-4931)
                    const std::string why = window_error(n);
                    if (!why.empty()) return fail("node " + std::to_string(n.id) + ": " + why);
                    continue;
                }
                case Op::ExtentWitness:
                    // checked on the host before the launches (build_plan);
                    // its value itself is read by nothing this build runs
                    if (!users[n.id].empty())
                        return fail("node " + std::to_string(n.id) + ": an ExtentWitness value read by a launch");
                    if (n.named_claims)
                        return fail("node " + std::to_string(n.id) +
                                    ": an ExtentWitness with named claims is not checked by this build");
                    continue;
                case Op::Sum: case Op::MaxReduce: case Op::MinReduce: case Op::ProdReduce: case Op::Argmax:
                case Op::Argmin: {
                    Region r;
                    r.kind = RegionKind::Reduce;
                    r.reduce_op = n.op == Op::Sum ? CHELIS_REDUCE_SUM : n.op == Op::MaxReduce ? CHELIS_REDUCE_MAX
                                  : n.op == Op::MinReduce ? CHELIS_REDUCE_MIN : n.op == Op::ProdReduce ? CHELIS_REDUCE_PROD
                                  : n.op == Op::Argmax ? CHELIS_REDUCE_ARGMAX : CHELIS_REDUCE_ARGMIN;
                    r.axis = n.axis;
                    r.in = {n.inputs[0]};
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::Count: {
                    if (n.axes.size() != 1)
                        return fail("node " + std::to_string(n.id) + ": Count over several axes is not built");
                    Region r;
                    r.kind = RegionKind::Count;
                    r.axis = n.axes[0];
                    r.in = {n.inputs[0]};
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::Softmax: {
                    if (n.axis != (int64_t)n.dims.size() - 1)
                        return fail("node " + std::to_string(n.id) + ": softmax over a leading axis is not built");
                    Region r;
                    r.kind = RegionKind::Softmax;
                    r.in = {n.inputs[0]};
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::Relu: case Op::ReluAdjoint: {
                    Region r;
                    r.kind = n.op == Op::Relu ? RegionKind::Relu : RegionKind::ReluAdjoint;
                    r.in = n.inputs;
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::Compare: {
                    const int code = compare_code(n.compare);
                    if (code < 0 || n.inputs.size() != 2)
                        return fail("node " + std::to_string(n.id) + ": Compare `" + n.compare + "` is not built");
                    single(n, RegionKind::Compare, code);
                    continue;
                }
                case Op::Logical: {
                    const int code = n.compare == "and" ? CHELIS_LOGICAL_AND : n.compare == "or" ? CHELIS_LOGICAL_OR
                                     : n.compare == "not" ? CHELIS_LOGICAL_NOT : -1;
                    if (code < 0 || n.inputs.size() != (code == CHELIS_LOGICAL_NOT ? 1u : 2u))
                        return fail("node " + std::to_string(n.id) + ": Logical `" + n.compare + "` is not built");
                    single(n, RegionKind::Logical, code);
                    continue;
                }
                case Op::Where:
                    if (n.inputs.size() != 3)
                        return fail("node " + std::to_string(n.id) + ": Where needs a condition and two branches");
                    single(n, RegionKind::Where);
                    continue;
                case Op::Cast:
                    if (n.inputs.size() != 1 || prim_width(n.cast_to) == 0 || n.cast_to == Prim::Key ||
                        N(n.inputs[0]).prec == Prim::Key)
                        return fail("node " + std::to_string(n.id) + ": a Cast this build has no conversion for");
                    single(n, RegionKind::Cast);
                    continue;
                case Op::Gather: {
                    if (n.inputs.size() != 2)
                        return fail("node " + std::to_string(n.id) + ": Gather needs values and indices");
                    Region r;
                    r.kind = RegionKind::Gather;
                    r.axis = n.axis;
                    r.batch_rank = n.batch_rank;
                    r.in = n.inputs;
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::Dropout: case Op::DropoutReplay: {
                    double rate;
                    Prim rp;
                    if (n.inputs.size() != 3 || !const_of(n.inputs[1], &rate, &rp))
                        return fail("node " + std::to_string(n.id) + ": dropout needs a constant rate and a key");
                    if (N(n.inputs[2]).prec != Prim::Key || !N(n.inputs[2]).dims.empty())
                        return fail("node " + std::to_string(n.id) + ": dropout's key must be one rank-0 key");
                    Region r;
                    r.kind = RegionKind::Dropout;
                    r.replay = n.op == Op::DropoutReplay;
                    r.rate = rate;
                    r.host_key = derived_key(n.inputs[2], &r.key);
                    r.in = r.host_key ? std::vector<int64_t>{n.inputs[0]} : std::vector<int64_t>{n.inputs[0], n.inputs[2]};
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::KeyFromSeed: case Op::SplitKey: case Op::FoldIn: {
                    // derived here; every reader is a draw that takes the key
                    // from the plan
                    uint64_t k;
                    if (!derived_key(n.id, &k))
                        return fail("node " + std::to_string(n.id) + ": " + n.variant +
                                    " of a run-time seed, index or key tensor is not derived by this build (the "
                                    "reference derives draw keys at emission only, emit.rs:3594-3653)");
                    for (int64_t u : users[n.id]) {
                        const Op uo = N(u).op;
                        if (uo != Op::SplitKey && uo != Op::FoldIn && uo != Op::UniformLike && uo != Op::Dropout &&
                            uo != Op::DropoutReplay)
                            return fail("node " + std::to_string(n.id) + ": a derived key read by " + N(u).variant);
                    }
                    if (std::find(g.roots.begin(), g.roots.end(), n.id) != g.roots.end())
                        return fail("node " + std::to_string(n.id) + ": a derived key as a result");
                    continue;
                }
                case Op::UniformLike: {
                    // inputs [template, low, high, key] (dag.rs:995-1005);
                    // literal bounds, a rank-0 key (emit.rs:3655-3700)
                    double lo, hi;
                    Prim lp, hp;
                    if (n.inputs.size() != 4 || !const_of(n.inputs[1], &lo, &lp) || !const_of(n.inputs[2], &hi, &hp))
                        return fail("node " + std::to_string(n.id) + ": uniform_like needs literal bounds and a key");
                    if (n.owner_activation >= 0)
                        return fail("node " + std::to_string(n.id) + ": a draw under an activation is not built");
                    if (N(n.inputs[3]).prec != Prim::Key || !N(n.inputs[3]).dims.empty())
                        return fail("node " + std::to_string(n.id) + ": uniform_like's key must be one rank-0 key");
                    Region r;
                    r.kind = RegionKind::Uniform;
                    r.low = lo;
                    r.high = hi;
                    r.host_key = derived_key(n.inputs[3], &r.key);
                    if (!r.host_key) r.in = {n.inputs[3]};
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::Cumsum: {
                    if (n.inputs.size() != 1)
                        return fail("node " + std::to_string(n.id) + ": Cumsum reads one tensor");
                    Region r;
                    r.kind = RegionKind::Scan;
                    r.axis = n.axis;
                    r.code = n.code;
                    r.in = n.inputs;
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::Bitwise:
                    if (!is_integer(n.prec) || n.inputs.size() != 2)
                        return fail("node " + std::to_string(n.id) + ": Bitwise needs two integer operands");
                    single(n, RegionKind::Integer, CHELIS_INT_BITAND + n.code);
                    continue;
                case Op::ScatterAdd: case Op::Scatter: case Op::ScatterElements: {
                    if (n.inputs.size() != 3)
                        return fail("node " + std::to_string(n.id) + ": " + n.variant +
                                    " reads target, indices and updates");
                    Region r;
                    r.kind = RegionKind::Scatter;
                    r.code = n.op == Op::Scatter ? 0 : n.op == Op::ScatterAdd ? 1 : 2;
                    r.axis = n.axis;
                    r.batch_rank = n.batch_rank;
                    r.in = n.inputs;
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::Pad: {
                    const std::string why = window_error(n);
                    if (!why.empty()) return fail("node " + std::to_string(n.id) + ": " + why);
                    if (n.const_prec != n.prec)
                        return fail("node " + std::to_string(n.id) + ": Pad's fill is not of the tensor's dtype");
                    Region r;
                    r.kind = RegionKind::Pad;
                    r.lo = n.lo;
                    r.fill = n.const_bits;
                    r.in = {n.inputs[0]};
                    r.out = n.id;
                    r.covers = {n.id};
                    claim(r);
                    continue;
                }
                case Op::ExtremaAdjoint:
                    if (n.inputs.size() != 3)
                        return fail("node " + std::to_string(n.id) + ": ExtremaAdjoint needs left, right and cotangent");
                    single(n, RegionKind::ExtremaAdjoint, n.code);
                    continue;
                default:
                    return fail("node " + std::to_string(n.id) + ": " + n.variant +
                                " is outside the region kinds this build runs");
            }
        }
        return true;
    }

    bool form(const std::vector<int64_t> &outputs) {
        if (!try_linreg(outputs)) try_mlp(outputs);
        for (const Node &n : g.nodes) {
            if (claimed[n.id] >= 0) continue;
            if (try_matmul(n.id)) continue;
            if (try_layer_norm(n.id)) continue;
            if (try_softmax(n.id)) continue;
            if (try_softmax_adjoint(n.id)) continue;
            if (try_gelu(n.id)) continue;
        }
        if (!generic()) return false;
        // keep launches in dependency order: by their result node
        std::vector<int> order(regions.size());
        for (size_t k = 0; k < order.size(); ++k) order[k] = (int)k;
        std::stable_sort(order.begin(), order.end(),
                         [&](int x, int y) { return regions[x].out < regions[y].out; });
        std::vector<Region> sorted;
        for (int k : order) sorted.push_back(regions[k]);
        regions.swap(sorted);
        for (size_t k = 0; k < regions.size(); ++k) {
            for (int64_t id : regions[k].covers)
                if (!free_leaf(id)) claimed[id] = (int)k;
            for (int64_t o : regions[k].outputs()) claimed[o] = (int)k;
        }
        return true;
    }
};

bool is_view_op(Op op) {
    return op == Op::Expand || op == Op::Permute || op == Op::Reshape || op == Op::Realize || op == Op::Copy ||
           op == Op::Store || op == Op::Shrink || op == Op::Stride;
}

// The reference's output specs (emit.rs:5901-5933): Store nodes in node
// order under their names, then the roots (the last node when there are
// none) as "root<index>", each node once.
void output_specs(const Graph &g, std::vector<int64_t> *nodes, std::vector<std::string> *labels) {
    std::set<int64_t> seen;
    for (const Node &n : g.nodes)
        if (n.op == Op::Store && seen.insert(n.id).second) {
            nodes->push_back(n.id);
            labels->push_back(n.name);
        }
    std::vector<int64_t> roots = g.roots;
    if (roots.empty() && !g.nodes.empty()) roots.push_back(g.nodes.back().id);
    for (size_t k = 0; k < roots.size(); ++k)
        if (seen.insert(roots[k]).second) {
            nodes->push_back(roots[k]);
            labels->push_back("root" + std::to_string(k));
        }
}

// The first extent this build cannot bind, as an error, or "".
std::string unbound_extent(const Node &n) {
    bool bad = false;
    for (int64_t d : n.dims) bad |= d == kUnboundExtent;
    if (n.op == Op::Expand) bad |= n.size == kUnboundExtent;
    if (n.op == Op::Reshape)
        for (int64_t d : n.new_shape) bad |= d == kUnboundExtent;
    if (!bad) return "";
    return "node " + std::to_string(n.id) + ": " + (n.extent_error.empty() ? "an unbound extent" : n.extent_error) +
           " is a run-time extent this build cannot bind";
}

// A materialized value's bytes: a literal, or coef * prod(symbols).
struct Size {
    int64_t coef = 0;
    std::vector<int64_t> symbols;
};
Size value_size(const Node &nd, int64_t width) {
    Size z;
    z.coef = width;
    for (int64_t d : nd.dims) {
        if (extent_is_symbol(d)) z.symbols.push_back(extent_symbol(d));
        else z.coef *= d;
    }
    std::sort(z.symbols.begin(), z.symbols.end());
    return z;
}

}  // namespace

bool build_plan(const Graph &input, Plan *plan, std::string *error) {
    *plan = Plan{};
    plan->graph = unfuse(input);
    const Graph &g = plan->graph;
    for (const Node &nd : g.nodes) {
        const std::string why = unbound_extent(nd);
        if (!why.empty()) {
            *error = why;
            return false;
        }
    }
    output_specs(g, &plan->output_nodes, &plan->output_labels);
    Planner P(g, plan->output_nodes);
    if (!P.form(plan->output_nodes)) {
        *error = P.error;
        return false;
    }
    // causal matmul modes: the scores product of a causal softmax skips the
    // tiles above the diagonal; the product reading the probabilities stops
    // each row tile's contraction at its last row
    for (Region &r : P.regions) {
        if (r.kind != RegionKind::MaskedSoftmax || !r.causal) continue;
        int64_t s = r.in[0];
        for (Region &m : P.regions)
            if (m.kind == RegionKind::Matmul && m.out == s && !m.has_bias && !m.has_residual &&
                m.activation == CHELIS_ACT_NONE && P.users[s].size() == 1 && !P.is_root[s])
                m.causal_mode = 1;
        for (Region &m : P.regions)
            if (m.kind == RegionKind::Matmul && m.in[0] == r.out && !m.has_bias && !m.has_residual &&
                m.activation == CHELIS_ACT_NONE && P.users[r.out].size() == 1 && !P.is_root[r.out])
                m.causal_mode = 2;
    }
    // causal attention: the scores product, the causal softmax over them and
    // the product reading the probabilities become one fused region when
    // the operands are binary32 [.., S, 64] with S a multiple of 64 (known
    // from the static extents); the scores and probabilities then never
    // reach memory
    for (size_t i = 0; i < P.regions.size(); ++i) {
        const Region &r = P.regions[i];
        if (r.kind != RegionKind::MaskedSoftmax || !r.causal) continue;
        int64_t m1 = -1, m2 = -1;
        for (size_t j = 0; j < P.regions.size(); ++j) {
            const Region &m = P.regions[j];
            if (m.kind == RegionKind::Matmul && m.causal_mode == 1 && m.out == r.in[0]) m1 = (int64_t)j;
            if (m.kind == RegionKind::Matmul && m.causal_mode == 2 && m.in[0] == r.out) m2 = (int64_t)j;
        }
        if (m1 < 0 || m2 < 0) continue;
        const Region &a = P.regions[m1], &b = P.regions[m2];
        const std::vector<int64_t> &qd = g.nodes[a.in[0]].dims, &kd = g.nodes[a.in[1]].dims,
                                   &vd = g.nodes[b.in[1]].dims, &od = g.nodes[b.out].dims;
        const size_t rk = qd.size();
        bool ok = rk >= 3 && kd.size() == rk && vd.size() == rk && od.size() == rk &&
                  g.nodes[a.in[0]].prec == Prim::F32 && g.nodes[a.in[1]].prec == Prim::F32 &&
                  g.nodes[b.in[1]].prec == Prim::F32 && g.nodes[b.out].prec == Prim::F32;
        for (size_t d = 0; ok && d < rk; ++d)
            ok = qd[d] > 0 && qd[d] == vd[d] && qd[d] == od[d] && (d + 2 < rk ? kd[d] == qd[d] : true);
        ok = ok && qd[rk - 1] == 64 && kd[rk - 2] == 64 && kd[rk - 1] == qd[rk - 2] && qd[rk - 2] % 64 == 0;
        if (!ok) continue;
        Region f;
        f.kind = RegionKind::Attention;
        f.out = b.out;
        f.in = {a.in[0], a.in[1], b.in[1]};
        f.scale = r.scale;
        for (const Region *part : {&a, &r, &b}) f.covers.insert(f.covers.end(), part->covers.begin(), part->covers.end());
        const size_t keep = (size_t)m2;
        std::vector<Region> next;
        for (size_t j = 0; j < P.regions.size(); ++j) {
            if (j == keep) next.push_back(f);
            else if (j != (size_t)m1 && j != i) next.push_back(P.regions[j]);
        }
        P.regions.swap(next);
        i = (size_t)-1;  // rescan from the start: indices moved
    }
    // products sharing their left operand, each with a bias and nothing
    // else after it, of one shape, whose weights and biases are available
    // where the first of them runs: one batched launch writing the results
    // back to back (the transformer's Q, K and V projections)
    {
        std::vector<bool> produced_before(g.nodes.size(), false);
        std::vector<Region> next;
        std::vector<bool> taken(P.regions.size(), false);
        auto plain = [&](const Region &r) {
            return r.kind == RegionKind::Matmul && r.has_bias && !r.has_residual && r.activation == CHELIS_ACT_NONE &&
                   !r.causal_mode && r.in.size() == 3 && !P.is_root[r.out] && g.nodes[r.out].count() > 0 &&
                   g.nodes[r.out].dims.size() == 2 && g.nodes[r.in[1]].dims.size() == 2;
        };
        for (size_t i = 0; i < P.regions.size(); ++i) {
            if (taken[i]) continue;
            const Region &r = P.regions[i];
            std::vector<size_t> members{i};
            if (plain(r)) {
                for (size_t j = i + 1; j < P.regions.size() && members.size() < (size_t)kMaxGroup; ++j) {
                    const Region &q = P.regions[j];
                    if (taken[j] || !plain(q) || q.in[0] != r.in[0] || g.nodes[q.out].dims != g.nodes[r.out].dims ||
                        g.nodes[q.out].prec != g.nodes[r.out].prec || g.nodes[q.in[1]].dims != g.nodes[r.in[1]].dims ||
                        g.nodes[q.in[2]].dims != g.nodes[r.in[2]].dims)
                        continue;
                    // its weight and bias exist before the group runs
                    bool ready = true;
                    for (size_t k = i; k < j && ready; ++k)
                        for (int64_t o : P.regions[k].outputs())
                            ready = ready && o != q.in[1] && o != q.in[2];
                    if (ready) members.push_back(j);
                }
            }
            if (members.size() < 2) {
                next.push_back(r);
                continue;
            }
            Region grp;
            grp.kind = RegionKind::MatmulGroup;
            grp.out = r.out;
            grp.in = {r.in[0]};
            for (size_t m : members) {
                taken[m] = true;
                const Region &q = P.regions[m];
                if (m != i) grp.more_out.push_back(q.out);
                grp.in.push_back(q.in[1]);
                grp.in.push_back(q.in[2]);
                grp.covers.insert(grp.covers.end(), q.covers.begin(), q.covers.end());
            }
            next.push_back(grp);
        }
        P.regions.swap(next);
    }
    plan->regions = P.regions;
    const size_t n = g.nodes.size();
    plan->values.assign(n, ValueInfo{});
    std::vector<bool> produced(n, false);
    for (const Region &r : plan->regions)
        for (int64_t o : r.outputs()) produced[o] = true;
    // caller inputs: one slot per Load name (a repeated Load aliases it,
    // emit.rs:5881-5892), in first-appearance order
    std::map<std::string, int64_t> input_slot;
    for (const Node &nd : g.nodes) {
        ValueInfo &v = plan->values[nd.id];
        if (nd.op == Op::Load) {
            v.storage = Storage::Input;
            auto it = input_slot.find(nd.name);
            if (it == input_slot.end()) {
                v.input = (int64_t)plan->input_nodes.size();
                input_slot[nd.name] = v.input;
                plan->input_nodes.push_back(nd.id);
                plan->input_labels.push_back(nd.name);
            } else {
                const Node &first = g.nodes[plan->input_nodes[it->second]];
                if (first.dims != nd.dims || first.prec != nd.prec) {
                    *error = "node " + std::to_string(nd.id) + ": Load `" + nd.name +
                             "` repeats an input name with another type";
                    return false;
                }
                v.input = it->second;
            }
        } else if (nd.op == Op::Const) {
            v.storage = Storage::Const;
            v.const_index = (int64_t)plan->const_bits.size();
            plan->const_bits.push_back(nd.const_bits);
            plan->const_prec.push_back(nd.const_prec);
        } else if (nd.op == Op::ConstTensor) {
            // the literal's bytes in the pool, whole 8-byte cells (unmasked)
            v.storage = Storage::Const;
            v.const_dense = true;
            v.const_index = (int64_t)plan->const_bits.size();
            for (uint64_t cell : nd.tensor_cells) {
                plan->const_bits.push_back(cell);
                plan->const_prec.push_back(Prim::Int64);
            }
        } else if (produced[nd.id]) {
            v.storage = Storage::Slot;
        } else if (is_view_op(nd.op) && P.claimed[nd.id] < 0) {
            v.storage = Storage::View;
            v.base = nd.inputs[0];
        } else {
            v.storage = Storage::Inlined;
        }
    }
    // run-time extents: each symbol is read from the first input axis that
    // declares it (inputs in slot order, axes in order); later declaring
    // axes must agree (emit.rs:1141-1168)
    std::vector<bool> bound(g.symbols.size(), false);
    for (size_t slot = 0; slot < plan->input_nodes.size(); ++slot) {
        const Node &ld = g.nodes[plan->input_nodes[slot]];
        for (size_t a = 0; a < ld.dims.size(); ++a) {
            if (!extent_is_symbol(ld.dims[a])) continue;
            const int64_t sym = extent_symbol(ld.dims[a]);
            SymbolRead r{sym, (int64_t)slot, (int64_t)a};
            if (bound[sym]) {
                plan->checks.push_back(r);
            } else {
                bound[sym] = true;
                plan->binds.push_back(r);
                plan->symbolic_dims.push_back(sym);
            }
        }
    }
    for (const Node &nd : g.nodes) {
        std::vector<int64_t> ext = nd.dims;
        if (nd.op == Op::Expand) ext.push_back(nd.size);
        if (nd.op == Op::Reshape) ext.insert(ext.end(), nd.new_shape.begin(), nd.new_shape.end());
        for (int64_t e : ext)
            if (extent_is_symbol(e) && !bound[extent_symbol(e)]) {
                *error = "node " + std::to_string(nd.id) + ": run-time extent `" + g.symbols[extent_symbol(e)] +
                         "` is not declared by any input";
                return false;
            }
    }
    // ExtentWitness requirements, checked on the host before the launches
    for (const Node &nd : g.nodes) {
        if (nd.op != Op::ExtentWitness || nd.site == WitnessSite::LiteralResultClaim || nd.requirements.empty())
            continue;
        auto it = input_slot.find(nd.name);
        const Node *ld = it == input_slot.end() ? nullptr : &g.nodes[plan->input_nodes[it->second]];
        if (!ld || nd.axis < 0 || nd.axis >= (int64_t)ld->dims.size()) {
            *error = "node " + std::to_string(nd.id) + ": ExtentWitness reads `" + nd.name +
                     "`, which is no input axis of this program";
            return false;
        }
        for (int64_t req : nd.requirements) plan->extent_checks.push_back({it->second, nd.axis, req, nd.name});
    }
    // every region input must have storage
    for (const Region &r : plan->regions)
        for (int64_t in : r.in)
            if (plan->values[in].storage == Storage::Inlined) {
                *error = "node " + std::to_string(in) + " is read by a launch but computed inside another";
                return false;
            }
    // outputs: a region result is written straight into the caller's
    // output (through a reshape or store view when the output is one);
    // anything else is copied there by a last launch
    std::vector<bool> grouped(n, false);
    for (const Region &r : plan->regions)
        if (r.kind == RegionKind::MatmulGroup)
            for (int64_t o : r.outputs()) grouped[o] = true;
    for (size_t o = 0; o < plan->output_nodes.size(); ++o) {
        const int64_t root = plan->output_nodes[o];
        int64_t v = root;
        while (plan->values[v].storage == Storage::View &&
               (g.nodes[v].op == Op::Reshape || g.nodes[v].op == Op::Store) && P.users[v].size() <= 1 &&
               P.users[plan->values[v].base].size() == 1 && !P.is_root[plan->values[v].base])
            v = plan->values[v].base;
        ValueInfo &vi = plan->values[v];
        if (vi.storage == Storage::Slot && vi.output < 0 && !grouped[v] && (v == root || P.users[v].size() == 1)) {
            vi.storage = Storage::Output;
            vi.output = (int64_t)o;
            vi.base = root;  // the packet is the output's, viewed with this node's shape
        } else {
            Region c;
            c.kind = RegionKind::Copy;
            c.in = {root};
            c.out = root;
            c.axis = (int64_t)o;  // the output slot
            plan->regions.push_back(c);
        }
    }
    // a materialized value read only through one Permute is stored in the
    // permuted order, so the permuted view is dense (a later Reshape of it
    // is then a view too); matmul results (their launcher writes any strided
    // layout) and attention results whose permutation keeps the head axis
    // innermost (the fused kernel writes rows of 64 contiguous values)
    for (const Region &r : plan->regions) {
        if (r.kind != RegionKind::Matmul && r.kind != RegionKind::Attention) continue;
        ValueInfo &vi = plan->values[r.out];
        if (vi.storage != Storage::Slot || P.users[r.out].size() != 1) continue;
        const Node &u = g.nodes[P.users[r.out][0]];
        const size_t rk = g.nodes[r.out].dims.size();
        if (u.op != Op::Permute || u.axes.size() != rk) continue;
        if (r.kind == RegionKind::Attention && u.axes[rk - 1] != (int64_t)rk - 1) continue;
        vi.layout = u.axes;
    }
    // slot plan: lifetimes in launch order, views charged to their base.
    // A literal value takes the free literal range that fits it best (or
    // grows the largest); a value sized by run-time extents reuses a free
    // range only of the same size expression (the reference's exact-capacity
    // reuse, memory.rs:32-182), so every range has one formula.
    std::vector<int64_t> last(n, -1);
    for (size_t k = 0; k < plan->regions.size(); ++k) {
        for (int64_t in : plan->regions[k].in) {
            int64_t b = in;
            while (plan->values[b].storage == Storage::View) b = plan->values[b].base;
            last[b] = std::max(last[b], (int64_t)k);
        }
    }
    std::vector<Slot> slots;
    std::vector<bool> busy;
    std::vector<std::vector<int64_t>> release_at(plan->regions.size());
    for (size_t k = 0; k < plan->regions.size(); ++k) {
        const Region &r = plan->regions[k];
        // a matmul group's results share one range, back to back
        const bool group = r.kind == RegionKind::MatmulGroup;
        const std::vector<int64_t> results = r.kind == RegionKind::Copy ? std::vector<int64_t>{} : r.outputs();
        for (size_t ri = 0; ri < results.size() && (!group || ri == 0); ++ri) {
            const int64_t out = results[ri];
            if (plan->values[out].storage != Storage::Slot) continue;
            ValueInfo &vi = plan->values[out];
            const Node &nd = g.nodes[out];
            const int64_t width = r.kind == RegionKind::Reduce && (r.reduce_op == CHELIS_REDUCE_ARGMAX ||
                                                                   r.reduce_op == CHELIS_REDUCE_ARGMIN)
                                      ? 8
                                      : (r.kind == RegionKind::Count ? 8 : prim_width(nd.prec));
            Size z = value_size(nd, width);
            int64_t end = std::max(last[out], (int64_t)k);
            if (group) {
                for (size_t m = 0; m < results.size(); ++m) {
                    ValueInfo &mv = plan->values[results[m]];
                    mv.slot_offset = (int64_t)m * z.coef;  // literal extents (a group requires them)
                    end = std::max(end, last[results[m]]);
                }
                z.coef *= (int64_t)results.size();
            }
            int64_t best = -1;
            if (z.symbols.empty()) {
                const int64_t need = (z.coef + 255) & ~int64_t(255);
                for (size_t s = 0; s < slots.size(); ++s)
                    if (!busy[s] && !slots[s].symbolic() && slots[s].bytes >= need &&
                        (best < 0 || slots[s].bytes < slots[best].bytes))
                        best = (int64_t)s;
                if (best < 0)
                    for (size_t s = 0; s < slots.size(); ++s)
                        if (!busy[s] && !slots[s].symbolic() && (best < 0 || slots[s].bytes > slots[best].bytes))
                            best = (int64_t)s;
                if (best < 0) {
                    best = (int64_t)slots.size();
                    slots.push_back(Slot{});
                    busy.push_back(false);
                }
                slots[best].bytes = std::max(slots[best].bytes, need);
            } else {
                for (size_t s = 0; s < slots.size() && best < 0; ++s)
                    if (!busy[s] && slots[s].symbolic() && slots[s].coef == z.coef && slots[s].symbols == z.symbols)
                        best = (int64_t)s;
                if (best < 0) {
                    best = (int64_t)slots.size();
                    Slot sl;
                    sl.coef = z.coef;
                    sl.symbols = z.symbols;
                    slots.push_back(sl);
                    busy.push_back(false);
                }
            }
            busy[best] = true;
            vi.slot = best;
            if (group)
                for (int64_t o : results) plan->values[o].slot = best;
            release_at[end].push_back(best);
        }
        for (int64_t s : release_at[k]) busy[s] = false;
    }
    bool symbolic = false;
    int64_t off = 0;
    for (Slot &sl : slots) {
        symbolic |= sl.symbolic();
        sl.offset = off;
        off += sl.bytes;
        plan->slots.push_back(sl);
    }
    // the constant pool holds one 8-byte cell per constant
    plan->workspace_bytes = symbolic ? -1 : off;
    plan->peak_device_bytes = symbolic ? -1 : plan->workspace_bytes + 8 * (int64_t)plan->const_bits.size();
    return true;
}

std::vector<int64_t> resolve_dims(const std::vector<int64_t> &dims, const std::vector<int64_t> &values) {
    std::vector<int64_t> out(dims.size());
    for (size_t a = 0; a < dims.size(); ++a) out[a] = resolve_extent(dims[a], values);
    return out;
}

bool bind_symbols(const Plan &plan, const int64_t *const *input_shapes, const int32_t *input_ranks,
                  std::vector<int64_t> *values, std::string *error) {
    const Graph &g = plan.graph;
    values->assign(g.symbols.size(), 0);
    for (const SymbolRead &r : plan.binds) {
        if (r.axis >= input_ranks[r.input]) {
            *error = "input `" + plan.input_labels[r.input] + "` has no axis " + std::to_string(r.axis);
            return false;
        }
        const int64_t e = input_shapes[r.input][r.axis];
        if (e < 0) {
            *error = "input `" + plan.input_labels[r.input] + "` axis " + std::to_string(r.axis) +
                     " is negative";
            return false;
        }
        (*values)[r.symbol] = e;
    }
    for (const SymbolRead &r : plan.checks) {
        const int64_t e = r.axis < input_ranks[r.input] ? input_shapes[r.input][r.axis] : -1;
        if (e != (*values)[r.symbol]) {
            *error = "symbolic dim `" + g.symbols[r.symbol] + "` mismatch: " + plan.input_labels[r.input] + "[" +
                     std::to_string(r.axis) + "]=" + std::to_string(e) + " but " + g.symbols[r.symbol] + "=" +
                     std::to_string((*values)[r.symbol]);
            return false;
        }
    }
    return true;
}

bool layout_slots(const Plan &plan, const std::vector<int64_t> &values, std::vector<int64_t> *offsets,
                  int64_t *workspace) {
    offsets->assign(plan.slots.size(), 0);
    int64_t off = 0;
    const int64_t limit = int64_t(1) << 62;
    for (size_t k = 0; k < plan.slots.size(); ++k) {
        const Slot &sl = plan.slots[k];
        int64_t bytes = sl.bytes;
        if (sl.symbolic()) {
            bytes = sl.coef;
            for (int64_t s : sl.symbols) {
                const int64_t v = values[(size_t)s];
                if (v != 0 && bytes > limit / v) return false;
                bytes *= v;
            }
            bytes = (bytes + 255) & ~int64_t(255);
        }
        (*offsets)[k] = off;
        if (off > limit - bytes) return false;
        off += bytes;
    }
    *workspace = off;
    return true;
}

std::string peak_formula(const Plan &plan) {
    std::string f;
    auto term = [&](const std::string &t) { f += (f.empty() ? "" : " + ") + t; };
    for (const Slot &sl : plan.slots) {
        if (!sl.symbolic()) {
            term(std::to_string(sl.bytes));
            continue;
        }
        std::string t = std::to_string(sl.coef);
        for (int64_t s : sl.symbols) t += "*" + plan.graph.symbols[(size_t)s];
        term(sl.coef % 256 == 0 ? t : "round_up(" + t + ", 256)");
    }
    if (!plan.const_bits.empty()) term(std::to_string(8 * plan.const_bits.size()));
    return f.empty() ? "0" : f;
}

std::string describe_plan(const Plan &plan) {
    std::string s;
    for (size_t k = 0; k < plan.regions.size(); ++k) {
        const Region &r = plan.regions[k];
        s += std::to_string(k) + " " + region_kind_name(r.kind) + " out=" + std::to_string(r.out);
        if (!r.more_out.empty()) {
            s += "+[";
            for (size_t i = 0; i < r.more_out.size(); ++i) s += (i ? "," : "") + std::to_string(r.more_out[i]);
            s += "]";
        }
        s += " in=[";
        for (size_t i = 0; i < r.in.size(); ++i) s += (i ? "," : "") + std::to_string(r.in[i]);
        s += "]";
        if (r.kind == RegionKind::Chain || (r.kind == RegionKind::Reduce && r.has_chain))
            s += " steps=" + std::to_string(r.chain.n_steps);
        if (r.kind == RegionKind::Reduce) s += " op=" + std::to_string(r.reduce_op) + " axis=" + std::to_string(r.axis);
        if (r.kind == RegionKind::Matmul) {
            if (r.has_bias) s += " bias";
            if (r.activation == CHELIS_ACT_RELU) s += " relu";
            if (r.activation == CHELIS_ACT_GELU) s += " gelu";
            if (r.has_residual) s += " residual";
            if (r.causal_mode) s += " causal=" + std::to_string(r.causal_mode);
            if (!plan.values[r.out].layout.empty()) s += " permuted";
        }
        if (r.kind == RegionKind::MaskedSoftmax || r.kind == RegionKind::Attention) s += " causal";
        if (r.kind == RegionKind::Attention && !plan.values[r.out].layout.empty()) s += " permuted";
        const ValueInfo &v = plan.values[r.out];
        if (r.kind != RegionKind::Copy) {
            if (v.storage == Storage::Output) s += " -> output " + std::to_string(v.output);
            else if (v.storage == Storage::Slot) s += " -> slot " + std::to_string(v.slot);
        } else {
            s += " -> output " + std::to_string(r.axis);
        }
        s += "\n";
    }
    return s;
}

}  // namespace dag
}  // namespace chelis

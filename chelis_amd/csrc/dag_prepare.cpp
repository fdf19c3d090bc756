// prepare_dag_for_codegen (crates/chelis-backend-hip/src/lib.rs:173-227):
// the HIP backend's BLAS selection before codegen. A lowered matmul
//   [Cast bf16/f16](Sum{L+1}(Mul(Expand{L+2}(a), Expand{L}(b))))
// becomes one BlasMatmul{batch_dims, m, n, k, accumulator} node over a and
// b, under the recognizer's conditions (crates/chelis-ir-core/src/
// specialize.rs:150-226,623-793): a float result (f32 / f64, or bf16 / f16
// through the final Cast of an f32 sum), operand and product precisions
// equal to it, expands that insert exactly their declared extents, operands
// whose matrix slices are contiguous (no Permute on the way), no replaced
// node owning a result claim, and no zero extent. The swallowed Mul, Sum and
// Expand nodes are dropped once nothing else reads them.
//
// The reference then inserts a Realize copy before every BlasMatmul operand
// so hipBLAS sees dense storage (lib.rs:182-198). This build does not: its
// matmul dispatch reads any strided operand (16-byte loads along whichever
// axis is contiguous), so the copies would only cost traffic. The pass is
// idempotent, as the reference's is.
#include <algorithm>

#include "dag.h"

namespace chelis {
namespace dag {
namespace {

struct MatmulMatch {
    int64_t out = -1, sum = -1, mul = -1, ea = -1, eb = -1, a = -1, b = -1;
    std::vector<int64_t> batch;
    int64_t m = 0, n = 0, k = 0;
    Prim accumulator = Prim::Other;
};

// specialize.rs:795-900: whether a node's matrix slices are contiguous.
bool contiguous_slices(const Graph &g, int64_t id) {
    const Node &n = g.nodes[(size_t)id];
    switch (n.op) {
        case Op::Permute: case Op::ExtentWitness: case Op::Count: case Op::Other:
            return false;
        case Op::Reshape: case Op::Store:
            return !n.inputs.empty() && contiguous_slices(g, n.inputs[0]);
        case Op::Expand:
            return n.axis + 2 < (int64_t)n.dims.size() && !n.inputs.empty() && contiguous_slices(g, n.inputs[0]);
        default:
            return true;
    }
}

bool float_result(Prim p) { return p == Prim::F32 || p == Prim::F64 || p == Prim::Bf16 || p == Prim::F16; }

bool detect(const Graph &g, int64_t id, MatmulMatch *mm) {
    const Node &out = g.nodes[(size_t)id];
    if (!float_result(out.prec)) return false;
    int64_t sum = id;
    if (out.op == Op::Cast) {
        if ((out.cast_to != Prim::Bf16 && out.cast_to != Prim::F16) || out.inputs.size() != 1 ||
            out.cast_to != out.prec)
            return false;
        const Node &in = g.nodes[(size_t)out.inputs[0]];
        if (in.prec != Prim::F32 || in.dims != out.dims) return false;
        sum = out.inputs[0];
    }
    const Node &S = g.nodes[(size_t)sum];
    if (S.op != Op::Sum || S.inputs.size() != 1 || S.dims.size() < 2) return false;
    const int64_t L = (int64_t)S.dims.size() - 2;
    if (S.axis != L + 1) return false;
    const Node &M = g.nodes[(size_t)S.inputs[0]];
    if (M.op != Op::Mul || M.inputs.size() != 2) return false;
    const Node &EA = g.nodes[(size_t)M.inputs[0]], &EB = g.nodes[(size_t)M.inputs[1]];
    if (EA.op != Op::Expand || EB.op != Op::Expand || EA.axis != L + 2 || EB.axis != L) return false;
    // the expand inserts exactly its declared extent (specialize.rs:623-653)
    if (EA.size != EA.dims[(size_t)EA.axis] || EB.size != EB.dims[(size_t)EB.axis]) return false;
    const int64_t a = EA.inputs[0], b = EB.inputs[0];
    if (!contiguous_slices(g, a) || !contiguous_slices(g, b)) return false;
    const Node &A = g.nodes[(size_t)a], &B = g.nodes[(size_t)b];
    if (A.prec != out.prec || B.prec != out.prec || M.prec != A.prec) return false;
    if (A.dims.size() != (size_t)L + 2 || B.dims.size() != (size_t)L + 2) return false;
    std::vector<int64_t> batch(S.dims.begin(), S.dims.begin() + L);
    if (!std::equal(batch.begin(), batch.end(), A.dims.begin()) || !std::equal(batch.begin(), batch.end(), B.dims.begin()))
        return false;
    const int64_t m = A.dims[(size_t)L], k = A.dims[(size_t)L + 1], n = B.dims[(size_t)L + 1];
    if (B.dims[(size_t)L] != k) return false;
    std::vector<int64_t> expect = batch;
    expect.push_back(m);
    expect.push_back(n);
    if (S.dims != expect) return false;
    if (m == 0 || n == 0 || k == 0) return false;  // an empty contraction keeps its RISC form
    mm->out = id;
    mm->sum = sum;
    mm->mul = S.inputs[0];
    mm->ea = M.inputs[0];
    mm->eb = M.inputs[1];
    mm->a = a;
    mm->b = b;
    mm->batch = batch;
    mm->m = m;
    mm->n = n;
    mm->k = k;
    mm->accumulator = S.accumulator;
    return true;
}

std::string dim_expr(const Graph &g, int64_t e) {
    if (extent_is_symbol(e)) return "{\"Sym\":" + json_quote(g.symbols[(size_t)extent_symbol(e)]) + "}";
    return "{\"Concrete\":" + std::to_string(e) + "}";
}

void append_span(Node *n, const std::string &span) {
    if (n->has_span && n->span == span) return;
    if (std::find(n->merged_spans.begin(), n->merged_spans.end(), span) != n->merged_spans.end()) return;
    n->merged_spans.push_back(span);
    std::sort(n->merged_spans.begin(), n->merged_spans.end());
}

void append_provenance(Node *target, const Node &src) {
    if (src.has_span) append_span(target, src.span);
    for (const std::string &s : src.merged_spans) append_span(target, s);
}

}  // namespace

Graph prepare_for_codegen(const Graph &g) {
    const std::vector<bool> claimed = claimed_producers(g);
    const size_t n = g.nodes.size();
    std::vector<MatmulMatch> matches(n);
    std::vector<bool> replaced(n, false), swallowed(n, false);
    for (const Node &nd : g.nodes) {
        MatmulMatch mm;
        if (!detect(g, nd.id, &mm)) continue;
        bool free = true;
        for (int64_t r : {mm.out, mm.sum, mm.mul, mm.ea, mm.eb}) free = free && !claimed[(size_t)r];
        if (!free) continue;
        matches[(size_t)nd.id] = mm;
        replaced[(size_t)nd.id] = true;
        for (int64_t r : {mm.sum, mm.mul, mm.ea, mm.eb})
            if (r != mm.out) swallowed[(size_t)r] = true;
    }
    // readers once the replaced outputs read a and b directly; a swallowed
    // node nothing else reads is dropped (walked from the back, so a chain
    // of them goes together)
    std::vector<int64_t> readers(n, 0);
    std::vector<bool> keep(n, true);
    auto deps = [&](const Node &nd, auto &&fn) {
        if (replaced[(size_t)nd.id]) {
            fn(matches[(size_t)nd.id].a);
            fn(matches[(size_t)nd.id].b);
        } else {
            for (int64_t i : nd.inputs) fn(i);
        }
        for (int64_t i : nd.shape_deps) fn(i);
        for (int64_t i : nd.claim_deps) fn(i);
        if (nd.owner_activation >= 0) fn(nd.owner_activation);
    };
    for (const Node &nd : g.nodes) deps(nd, [&](int64_t i) { ++readers[(size_t)i]; });
    for (int64_t r : g.roots) ++readers[(size_t)r];
    for (size_t k = n; k-- > 0;) {
        const Node &nd = g.nodes[k];
        if (!swallowed[k] || readers[k] > 0 || nd.op == Op::Store) continue;
        keep[k] = false;
        deps(nd, [&](int64_t i) { --readers[(size_t)i]; });
    }
    Graph out;
    out.declarations = g.declarations;
    out.symbols = g.symbols;
    std::vector<int64_t> map(n, -1);
    for (const Node &nd : g.nodes) {
        if (!keep[(size_t)nd.id]) continue;
        Node c = nd;
        c.id = (int64_t)out.nodes.size();
        if (replaced[(size_t)nd.id]) {
            const MatmulMatch &mm = matches[(size_t)nd.id];
            c.op = Op::BlasMatmul;
            c.variant = "BlasMatmul";
            c.inputs = {mm.a, mm.b};
            c.cast_to = Prim::Other;
            c.reusable = -1;
            std::string op = "{\"BlasMatmul\":{\"batch_dims\":[";
            for (size_t d = 0; d < mm.batch.size(); ++d) op += (d ? "," : "") + dim_expr(g, mm.batch[d]);
            op += "],\"m\":" + dim_expr(g, mm.m) + ",\"n\":" + dim_expr(g, mm.n) + ",\"k\":" + dim_expr(g, mm.k) +
                  ",\"accumulator\":" + json_quote(prim_name(mm.accumulator)) + "}}";
            c.raw_op = op;
            c.merged_spans.clear();
            append_provenance(&c, nd);
            for (int64_t r : {mm.sum, mm.mul, mm.ea, mm.eb})
                if (r != nd.id) append_provenance(&c, g.nodes[(size_t)r]);
        }
        for (int64_t &i : c.inputs) i = map[(size_t)i];
        for (int64_t &i : c.shape_deps) i = map[(size_t)i];
        for (int64_t &i : c.claim_deps) i = map[(size_t)i];
        if (c.reusable >= 0) c.reusable = map[(size_t)c.reusable];
        if (c.owner_activation >= 0) c.owner_activation = map[(size_t)c.owner_activation];
        map[(size_t)nd.id] = c.id;
        out.nodes.push_back(std::move(c));
    }
    for (int64_t r : g.roots) out.roots.push_back(map[(size_t)r]);
    return out;
}

}  // namespace dag
}  // namespace chelis

// Chain fusion over the DAG, with the reference's rules
// (crates/chelis-dag-core/src/fuse.rs): it never duplicates work (a node
// with several consumers ends a chain), a chain holds only fusible float
// elementwise ops under one owner, and chains shorter than two nodes stay
// as they are. unfuse() writes a FusedElem back as its primitive nodes, so
// the region patterns see fused and unfused inputs in one form.
#include <algorithm>

#include "dag.h"

namespace chelis {
namespace dag {

std::vector<int64_t> consumer_counts(const Graph &g) {
    // DagNode::dependencies (crates/chelis-dag-core/src/dag.rs:2449-2456):
    // inputs, shape and claim dependencies and the owner's activation; each
    // root counts once more (fuse.rs:61-74).
    std::vector<int64_t> c(g.nodes.size(), 0);
    for (const Node &n : g.nodes) {
        for (int64_t i : n.inputs) ++c[i];
        for (int64_t i : n.shape_deps) ++c[i];
        for (int64_t i : n.claim_deps) ++c[i];
        if (n.owner_activation >= 0 && n.owner_activation < (int64_t)c.size()) ++c[n.owner_activation];
    }
    for (int64_t r : g.roots) ++c[r];
    return c;
}

bool is_integer(Prim p) {
    return p == Prim::Int8 || p == Prim::Int16 || p == Prim::Int32 || p == Prim::Int64;
}

namespace {

// DagView::is_activation_gated (crates/chelis-dag-core/src/dag.rs:2864-2880)
// over the chain ops: under an activation, an op whose run-time check may
// fail keeps its own kernel - integer add / sub / mul / neg / abs / floor
// and truncating division (operand values, dag.rs:2548-2551) and every
// division (an integer operand check, or a lowered mean's divisor,
// dag.rs:2555-2556).
bool activation_gated(const Node &n) {
    if (n.owner_activation < 0) return false;
    if (n.op == Op::Div) return true;
    if (!is_integer(n.prec)) return false;
    switch (n.op) {
        case Op::Add: case Op::Sub: case Op::Mul: case Op::Neg: case Op::Abs: case Op::FloorDiv:
        case Op::TruncDiv:
            return true;
        default:
            return false;
    }
}

// fuse.rs:76-96: fused_step_op's table, minus the integer forms that stay
// materialized (abs / sub / max / min) and the activation-gated ops.
bool fusible(const Node &n) {
    if (!op_is_chain_step(n.op)) return false;
    if (is_integer(n.prec) && (n.op == Op::Abs || n.op == Op::Sub || n.op == Op::MaxElem || n.op == Op::MinElem))
        return false;
    return !activation_gated(n);
}

bool owns_result_claim(const Graph &g, const Node &n) {
    auto claim = [&](int64_t dep) {
        const Node &w = g.nodes[(size_t)dep];
        return w.op == Op::ExtentWitness &&
               (w.site == WitnessSite::LiteralResultClaim || w.site == WitnessSite::ResultClaim ||
                w.site == WitnessSite::LocalAscriptionClaim);
    };
    for (int64_t d : n.shape_deps)
        if (claim(d)) return true;
    for (int64_t d : n.claim_deps)
        if (claim(d)) return true;
    return false;
}

}  // namespace

bool chain_fusible(const Node &n) { return fusible(n); }

std::vector<bool> claimed_producers(const Graph &g) {
    std::vector<bool> owned(g.nodes.size(), false);
    std::vector<int64_t> pending;
    for (const Node &n : g.nodes)
        if (owns_result_claim(g, n)) pending.push_back(n.id);
    while (!pending.empty()) {
        const int64_t cur = pending.back();
        pending.pop_back();
        if (owned[(size_t)cur]) continue;
        owned[(size_t)cur] = true;
        const Node &n = g.nodes[(size_t)cur];
        if ((n.op == Op::Copy || n.op == Op::Cast || n.op == Op::NamedCast) && !n.inputs.empty())
            pending.push_back(n.inputs[0]);
    }
    return owned;
}

Graph fuse(const Graph &g, std::vector<int64_t> *old_to_new) {
    const std::vector<int64_t> counts = consumer_counts(g);
    const size_t n = g.nodes.size();
    // first consumer (in node order) of each node through its inputs
    std::vector<std::vector<int64_t>> users(n);
    for (const Node &nd : g.nodes)
        for (int64_t i : nd.inputs)
            if (users[i].empty() || users[i].back() != nd.id) users[i].push_back(nd.id);
    // fuse.rs:136-191: walk in order, extend each start greedily forward
    std::vector<int64_t> chain_of(n, -1);
    std::vector<std::vector<int64_t>> chains;
    std::vector<bool> in_chain(n, false);
    // fuse.rs:147-161,183: a claimed producer is a barrier
    const std::vector<bool> barrier = claimed_producers(g);
    for (const Node &nd : g.nodes) {
        if (in_chain[nd.id] || !fusible(nd) || barrier[nd.id]) continue;
        std::vector<int64_t> chain{nd.id};
        in_chain[nd.id] = true;
        int64_t cur = nd.id;
        while (counts[cur] == 1) {
            int64_t next = -1;
            for (int64_t u : users[cur])
                if (!in_chain[u]) {
                    next = u;
                    break;
                }
            if (next < 0) break;
            const Node &c = g.nodes[next];
            if (!fusible(c) || barrier[next] || c.owner_decl != nd.owner_decl ||
                c.owner_activation != nd.owner_activation)
                break;
            chain.push_back(next);
            in_chain[next] = true;
            cur = next;
        }
        if (chain.size() >= 2) {
            for (int64_t id : chain) chain_of[id] = (int64_t)chains.size();
            chains.push_back(chain);
        } else {
            in_chain[nd.id] = false;  // a one-node "chain" stays an ordinary node
        }
    }
    // fuse.rs:206-332: rebuild, a chain becoming one FusedElem at its last node
    Graph out;
    out.declarations = g.declarations;
    out.symbols = g.symbols;
    std::vector<int64_t> map(n, -1);
    auto add = [&](Node node) {
        node.id = (int64_t)out.nodes.size();
        out.nodes.push_back(std::move(node));
        return out.nodes.back().id;
    };
    for (const Node &nd : g.nodes) {
        const int64_t ci = chain_of[nd.id];
        if (ci < 0) {
            Node copy = nd;
            for (int64_t &i : copy.inputs) i = map[i];
            for (int64_t &i : copy.shape_deps) i = map[i];
            for (int64_t &i : copy.claim_deps) i = map[i];
            if (copy.reusable >= 0) copy.reusable = map[copy.reusable];
            if (copy.owner_activation >= 0) copy.owner_activation = map[copy.owner_activation];
            map[nd.id] = add(std::move(copy));
            continue;
        }
        const std::vector<int64_t> &chain = chains[ci];
        if (nd.id != chain.back()) continue;
        // fuse.rs:373-421: external inputs in first-use order, steps in chain order
        Node f;
        f.op = Op::FusedElem;
        f.variant = "FusedElem";
        std::vector<int64_t> ext;
        for (size_t si = 0; si < chain.size(); ++si) {
            const Node &c = g.nodes[chain[si]];
            Step st;
            st.op = c.op;
            for (int64_t in : c.inputs) {
                auto pos = std::find(chain.begin(), chain.begin() + (long)si, in);
                if (pos != chain.begin() + (long)si) {
                    st.args.push_back(-(int)(pos - chain.begin()) - 1);
                } else {
                    auto e = std::find(ext.begin(), ext.end(), in);
                    if (e == ext.end()) {
                        ext.push_back(in);
                        e = ext.end() - 1;
                    }
                    st.args.push_back((int)(e - ext.begin()));
                }
            }
            f.steps.push_back(st);
        }
        for (int64_t e : ext) f.inputs.push_back(map[e]);
        const Node &last = g.nodes[chain.back()], &first = g.nodes[chain.front()];
        f.dims = last.dims;
        f.dims_raw = last.dims_raw;
        f.prec = last.prec;
        f.owner_decl = last.owner_decl;
        f.owner_activation = last.owner_activation >= 0 ? map[last.owner_activation] : -1;
        f.has_span = first.has_span;
        f.span = first.span;
        // fuse.rs:423-445: one reusable external input shared by the chain
        int64_t reuse = -1;
        bool clash = false;
        for (int64_t id : chain) {
            const int64_t r = g.nodes[id].reusable;
            if (r < 0 || std::find(ext.begin(), ext.end(), r) == ext.end()) continue;
            if (reuse < 0) reuse = r;
            else if (reuse != r) clash = true;
        }
        f.reusable = (reuse >= 0 && !clash) ? map[reuse] : -1;
        // merged spans: the first contributor's, then every other
        // contributor's span and merged spans, sorted and deduplicated
        std::vector<std::string> spans = first.merged_spans;
        for (size_t si = 1; si < chain.size(); ++si) {
            const Node &c = g.nodes[chain[si]];
            if (c.has_span) spans.push_back(c.span);
            spans.insert(spans.end(), c.merged_spans.begin(), c.merged_spans.end());
        }
        std::sort(spans.begin(), spans.end());
        spans.erase(std::unique(spans.begin(), spans.end()), spans.end());
        spans.erase(std::remove_if(spans.begin(), spans.end(),
                                   [&](const std::string &s) { return f.has_span && s == f.span; }),
                    spans.end());
        f.merged_spans = spans;
        for (int64_t id : chain) {
            for (int64_t d : g.nodes[id].shape_deps)
                if (std::find(f.shape_deps.begin(), f.shape_deps.end(), map[d]) == f.shape_deps.end())
                    f.shape_deps.push_back(map[d]);
            for (int64_t d : g.nodes[id].claim_deps)
                if (std::find(f.claim_deps.begin(), f.claim_deps.end(), map[d]) == f.claim_deps.end())
                    f.claim_deps.push_back(map[d]);
        }
        const int64_t nid = add(std::move(f));
        for (int64_t id : chain) map[id] = nid;
    }
    for (int64_t r : g.roots) out.roots.push_back(map[r]);
    if (old_to_new) *old_to_new = map;
    return out;
}

std::vector<bool> reduction_inlined(const Graph &g) {
    const std::vector<int64_t> counts = consumer_counts(g);
    std::vector<bool> inl(g.nodes.size(), false);
    for (const Node &nd : g.nodes) {
        if ((nd.op != Op::Sum && nd.op != Op::MaxReduce) || nd.inputs.empty()) continue;
        const int64_t in = nd.inputs[0];
        if (g.nodes[in].op == Op::FusedElem && counts[in] == 1) inl[in] = true;
    }
    return inl;
}

Graph unfuse(const Graph &g) {
    Graph out;
    out.declarations = g.declarations;
    out.symbols = g.symbols;
    std::vector<int64_t> map(g.nodes.size(), -1);
    for (const Node &nd : g.nodes) {
        if (nd.op != Op::FusedElem) {
            Node copy = nd;
            copy.id = (int64_t)out.nodes.size();
            for (int64_t &i : copy.inputs) i = map[i];
            for (int64_t &i : copy.shape_deps) i = map[i];
            for (int64_t &i : copy.claim_deps) i = map[i];
            if (copy.reusable >= 0) copy.reusable = map[copy.reusable];
            if (copy.owner_activation >= 0) copy.owner_activation = map[copy.owner_activation];
            map[nd.id] = copy.id;
            out.nodes.push_back(std::move(copy));
            continue;
        }
        std::vector<int64_t> step_ids;
        for (const Step &st : nd.steps) {
            Node p;
            p.id = (int64_t)out.nodes.size();
            p.op = st.op;
            p.variant = op_name(st.op);
            p.raw_op = json_quote(p.variant);
            for (int a : st.args) p.inputs.push_back(a >= 0 ? map[nd.inputs[a]] : step_ids[-a - 1]);
            p.dims = nd.dims;
            p.dims_raw = nd.dims_raw;
            p.prec = nd.prec;
            p.owner_decl = nd.owner_decl;
            p.owner_activation = nd.owner_activation >= 0 ? map[nd.owner_activation] : -1;
            step_ids.push_back(p.id);
            out.nodes.push_back(std::move(p));
        }
        Node &last = out.nodes.back();
        last.has_span = nd.has_span;
        last.span = nd.span;
        last.merged_spans = nd.merged_spans;
        for (int64_t d : nd.shape_deps) last.shape_deps.push_back(map[d]);
        for (int64_t d : nd.claim_deps) last.claim_deps.push_back(map[d]);
        map[nd.id] = last.id;
    }
    for (int64_t r : g.roots) out.roots.push_back(map[r]);
    return out;
}

}  // namespace dag
}  // namespace chelis

// The reference's DAG wire form read into chelis::dag::Graph and written
// back. Shapes follow serde's externally tagged enums over the types of
// crates/chelis-dag-core/src/dag.rs: a unit RiscOp is its variant name, any
// other is {"Variant": payload}; DimInfo is {"Lit": n} or {"Named": [name,
// n | null]}; RtDim is {"Lit": n}, {"Sym": name}, {"InputAxis": {"tensor": t,
// "axis": {"Lit": a}}}, {"Node": i} or "ToEnd"; a scalar is {"dtype": "f32", "bits": "<hex>"} or {"dtype": "int64",
// "value": n} (crates/chelis-numeric-core/src/dtype_semantics/wire_codec.rs:
// 488-512). Golden strings: crates/chelis-dag-core/tests/wire_behavior.rs:48,121.
//
// Extents (dag.rs:221-290): a literal; a run-time extent named by a symbol -
// DimInfo::Named(name, None) or RtDim::Sym(name) - bound from the input that
// declares it when the program runs; RtDim::InputAxis{tensor, axis}, the
// extent of that axis of the node's inputs[tensor] (literal or symbol);
// DimInfo::Named(name, Some(n)) is n. Bounds read from a node value
// (RtDim::Node), the to-the-end sentinel and DimExpr products or quotients
// are kept for the write-back and refused by the planner.
#include <cmath>
#include <cstring>

#include "dag.h"

namespace chelis {
namespace dag {

namespace {

struct OpName {
    const char *name;
    Op op;
};
const OpName kOps[] = {
    {"Load", Op::Load}, {"Const", Op::Const}, {"Iota", Op::Iota},
    {"Add", Op::Add}, {"Sub", Op::Sub}, {"Mul", Op::Mul}, {"Div", Op::Div}, {"Pow", Op::Pow},
    {"FloorDiv", Op::FloorDiv}, {"TruncDiv", Op::TruncDiv}, {"MaxElem", Op::MaxElem}, {"MinElem", Op::MinElem},
    {"Neg", Op::Neg}, {"Recip", Op::Recip}, {"Exp", Op::Exp}, {"Log", Op::Log}, {"Sin", Op::Sin},
    {"Sqrt", Op::Sqrt}, {"Cos", Op::Cos}, {"Tan", Op::Tan}, {"Atan", Op::Atan}, {"Tanh", Op::Tanh},
    {"Erf", Op::Erf}, {"Erfc", Op::Erfc}, {"Abs", Op::Abs}, {"Floor", Op::Floor}, {"Ceil", Op::Ceil},
    {"Round", Op::Round}, {"Relu", Op::Relu}, {"ReluAdjoint", Op::ReluAdjoint}, {"Where", Op::Where},
    {"Compare", Op::Compare}, {"Dropout", Op::Dropout}, {"DropoutReplay", Op::DropoutReplay}, {"Cast", Op::Cast},
    {"Sum", Op::Sum}, {"MaxReduce", Op::MaxReduce}, {"MinReduce", Op::MinReduce}, {"ProdReduce", Op::ProdReduce},
    {"Argmax", Op::Argmax}, {"Argmin", Op::Argmin}, {"Count", Op::Count}, {"Softmax", Op::Softmax},
    {"Expand", Op::Expand}, {"Permute", Op::Permute}, {"Reshape", Op::Reshape}, {"Realize", Op::Realize},
    {"Copy", Op::Copy}, {"FusedElem", Op::FusedElem}, {"BlasMatmul", Op::BlasMatmul},
    {"Store", Op::Store}, {"ExtentWitness", Op::ExtentWitness}, {"NamedCast", Op::NamedCast},
    {"Logical", Op::Logical}, {"Mod", Op::Mod}, {"Gather", Op::Gather},
    {"ExtremaAdjoint", Op::ExtremaAdjoint}, {"UniformLike", Op::UniformLike}, {"KeyFromSeed", Op::KeyFromSeed},
    {"Split", Op::SplitKey}, {"FoldIn", Op::FoldIn}, {"Cumsum", Op::Cumsum},
    {"Bitwise", Op::Bitwise}, {"Pad", Op::Pad}, {"Shrink", Op::Shrink}, {"Stride", Op::Stride},
    {"ScatterAdd", Op::ScatterAdd}, {"Scatter", Op::Scatter}, {"ScatterElements", Op::ScatterElements},
    {"ConstTensor", Op::ConstTensor}, {"Drop", Op::Drop},
};

struct PrimName {
    const char *wire;    // Prim's serde name (output_type.precision)
    const char *scalar;  // the scalar codec's dtype tag
    Prim prim;
};
const PrimName kPrims[] = {
    {"F32", "f32", Prim::F32}, {"F64", "f64", Prim::F64}, {"F16", "f16", Prim::F16},
    {"Bf16", "bf16", Prim::Bf16}, {"Int8", "int8", Prim::Int8}, {"Int16", "int16", Prim::Int16},
    {"Int32", "int32", Prim::Int32}, {"Int64", "int64", Prim::Int64}, {"Bool", "bool", Prim::Bool},
    {"Key", "key", Prim::Key},
};

Op op_of(const std::string &name) {
    for (const OpName &o : kOps)
        if (name == o.name) return o.op;
    return Op::Other;
}

bool prim_of(const Json *j, Prim *p) {
    if (!j || j->kind != Json::String) return false;
    for (const PrimName &q : kPrims)
        if (j->text == q.wire) {
            *p = q.prim;
            return true;
        }
    *p = Prim::Other;
    return true;  // a dtype this build has no kernels for: kept, refused later
}

bool int_of(const Json *j, int64_t *v) {
    if (!j || !j->is_int()) return false;
    *v = j->as_int();
    return true;
}

bool ids_of(const Json *j, std::vector<int64_t> *out) {
    out->clear();
    if (!j) return true;  // optional lists default to empty
    if (j->kind != Json::Array) return false;
    for (const Json &e : j->items) {
        int64_t v;
        if (!int_of(&e, &v)) return false;
        out->push_back(v);
    }
    return true;
}

// RtDim / DimInfo / DimExpr (dag.rs:221-290) as an extent code of `n`,
// whose inputs are already read. Unbindable forms give kUnboundExtent and
// set n->extent_error; malformed ones return false.
bool extent_of(const Json &j, Graph *g, Node *n, int64_t *code) {
    auto unbound = [&](const char *why) {
        if (n->extent_error.empty()) n->extent_error = why;
        *code = kUnboundExtent;
        return true;
    };
    if (j.kind == Json::String) {
        if (j.text == "ToEnd") return unbound("the to-the-end bound of a shrink");
        return false;
    }
    if (j.kind != Json::Object || j.fields.size() != 1) return false;
    const std::string &tag = j.fields[0].first;
    const Json &v = j.fields[0].second;
    if (tag == "Lit" || tag == "Concrete") {
        if (!v.is_int() || v.as_int() < 0) return false;
        *code = v.as_int();
        return true;
    }
    if (tag == "Named") {
        if (v.kind != Json::Array || v.items.size() != 2 || v.items[0].kind != Json::String) return false;
        if (v.items[1].is_int() && v.items[1].as_int() >= 0) {
            *code = v.items[1].as_int();
            return true;
        }
        if (v.items[1].kind != Json::Null) return false;
        *code = symbol_extent(g->symbol(v.items[0].text));
        return true;
    }
    if (tag == "Sym") {
        if (v.kind != Json::String) return false;
        *code = symbol_extent(g->symbol(v.text));
        return true;
    }
    if (tag == "InputAxis") {
        const Json *t = v.get("tensor"), *ax = v.get("axis");
        if (!t || !t->is_int() || !ax || ax->kind != Json::Object || ax->fields.size() != 1 ||
            ax->fields[0].first != "Lit" || !ax->fields[0].second.is_int())
            return false;
        const int64_t ti = t->as_int(), a = ax->fields[0].second.as_int();
        if (ti < 0 || ti >= (int64_t)n->inputs.size()) return false;
        const Node &src = g->nodes[(size_t)n->inputs[(size_t)ti]];
        if (a < 0 || a >= (int64_t)src.dims.size()) return false;
        *code = src.dims[(size_t)a];
        if (*code == kUnboundExtent) return unbound("an extent read from an unbound axis");
        return true;
    }
    if (tag == "Node") return unbound("a bound read from a node value");
    if (tag == "Mul" || tag == "Div") return unbound("a product or quotient of run-time extents");
    return false;
}

uint64_t hex_bits(const std::string &t, bool *ok) {
    uint64_t v = 0;
    *ok = !t.empty() && t.size() <= 16;
    for (char c : t) {
        v <<= 4;
        if (c >= '0' && c <= '9') v |= (uint64_t)(c - '0');
        else if (c >= 'a' && c <= 'f') v |= (uint64_t)(c - 'a' + 10);
        else *ok = false;
    }
    return v;
}

bool scalar_of(const Json *j, Node *n) {
    if (!j || j->kind != Json::Object) return false;
    const Json *dt = j->get("dtype");
    if (!dt || dt->kind != Json::String) return false;
    for (const PrimName &q : kPrims) {
        if (dt->text != q.scalar) continue;
        n->const_prec = q.prim;
        if (const Json *bits = j->get("bits")) {
            bool ok = bits->kind == Json::String;
            n->const_bits = ok ? hex_bits(bits->text, &ok) : 0;
            return ok && prim_is_float(q.prim);
        }
        const Json *v = j->get("value");
        if (!v) return false;
        if (v->kind == Json::Bool) {
            n->const_bits = v->boolean ? 1 : 0;
            return q.prim == Prim::Bool;
        }
        int64_t iv;
        if (!int_of(v, &iv)) return false;
        n->const_bits = (uint64_t)iv;
        return true;
    }
    return false;
}

bool step_op_of(const Json &j, Step *s) {
    const Json *op = j.get("op");
    const Json *ins = j.get("input_indices");
    if (!op || op->kind != Json::String || !ins || ins->kind != Json::Array) return false;
    s->op = op_of(op->text);
    if (!op_is_chain_step(s->op)) return false;
    for (const Json &in : ins->items) {
        if (in.kind != Json::Object || in.fields.size() != 1 || !in.fields[0].second.is_int()) return false;
        const int64_t k = in.fields[0].second.as_int();
        if (in.fields[0].first == "External") s->args.push_back((int)k);
        else if (in.fields[0].first == "PreviousStep") s->args.push_back(-(int)k - 1);
        else return false;
    }
    return true;
}

bool read_op(const Json &op, Graph *g, Node *n, std::string *why) {
    std::string raw;
    write_json(op, &raw);
    n->raw_op = raw;
    if (op.kind == Json::String) {
        n->variant = op.text;
        n->op = op_of(op.text);
        return true;
    }
    if (op.kind != Json::Object || op.fields.size() != 1) {
        *why = "op is neither a variant name nor a one-field object";
        return false;
    }
    const std::string &var = op.fields[0].first;
    const Json &p = op.fields[0].second;
    n->variant = var;
    n->op = op_of(var);
    switch (n->op) {
        case Op::Load:
        case Op::Store: {
            const Json *name = p.get("name");
            if (!name || name->kind != Json::String) return (*why = var + " without a name", false);
            n->name = name->text;
            return true;
        }
        case Op::ExtentWitness: {
            const Json *site = p.get("site"), *param = p.get("parameter"), *axis = p.get("axis"),
                       *reqs = p.get("requirements"), *claims = p.get("claims");
            if (!param || param->kind != Json::String || !axis || axis->kind != Json::Object ||
                axis->fields.size() != 1 || !axis->fields[0].second.is_int() || !reqs || reqs->kind != Json::Array)
                return (*why = "ExtentWitness needs parameter, axis and requirements", false);
            n->name = param->text;
            n->axis = axis->fields[0].second.as_int();
            for (const Json &r : reqs->items) {
                Node tmp;
                if (!scalar_of(&r, &tmp) || prim_is_float(tmp.const_prec))
                    return (*why = "ExtentWitness requirement is not an integer scalar", false);
                n->requirements.push_back((int64_t)tmp.const_bits);
            }
            n->named_claims = (claims && claims->kind == Json::Array) ? (int64_t)claims->items.size() : 0;
            n->site = WitnessSite::Other;
            if (site && site->kind == Json::String && site->text == "LiteralResultClaim")
                n->site = WitnessSite::LiteralResultClaim;
            else if (site && site->kind == Json::Object && site->fields.size() == 1) {
                if (site->fields[0].first == "ResultClaim") n->site = WitnessSite::ResultClaim;
                if (site->fields[0].first == "LocalAscriptionClaim") n->site = WitnessSite::LocalAscriptionClaim;
            }
            return true;
        }
        case Op::Const:
            if (!scalar_of(p.get("value"), n)) return (*why = "Const with an unreadable scalar", false);
            return true;
        case Op::ConstTensor: {
            // TensorStorage (dtype_semantics/wire_codec.rs:472-482): {"dtype":
            // tag, "bits": [hex...]} for floats, {"dtype": tag, "values":
            // [...]} for integers and bools
            const Json *d = p.get("data");
            const Json *dt = d ? d->get("dtype") : nullptr;
            if (!dt || dt->kind != Json::String) return (*why = "ConstTensor with unreadable data", false);
            const PrimName *q = nullptr;
            for (const PrimName &c : kPrims)
                if (dt->text == c.scalar) q = &c;
            if (!q || q->prim == Prim::Key) return (*why = "ConstTensor of dtype `" + dt->text + "`", false);
            n->const_prec = q->prim;
            const int64_t w = prim_width(q->prim);
            const Json *items = d->get(prim_is_float(q->prim) ? "bits" : "values");
            if (!items || items->kind != Json::Array) return (*why = "ConstTensor with unreadable data", false);
            const size_t count = items->items.size();
            n->tensor_cells.assign((count * (size_t)w + 7) / 8, 0);
            for (size_t k = 0; k < count; ++k) {
                const Json &e = items->items[k];
                uint64_t v = 0;
                bool ok = true;
                if (prim_is_float(q->prim)) {
                    ok = e.kind == Json::String;
                    if (ok) v = hex_bits(e.text, &ok);
                } else if (e.kind == Json::Bool) {
                    v = e.boolean ? 1 : 0;
                } else {
                    int64_t iv = 0;
                    ok = int_of(&e, &iv);
                    v = (uint64_t)iv;
                }
                if (!ok) return (*why = "ConstTensor element " + std::to_string(k) + " is unreadable", false);
                for (int64_t b = 0; b < w; ++b) {
                    const size_t byte = k * (size_t)w + (size_t)b;
                    n->tensor_cells[byte / 8] |= ((v >> (8 * b)) & 0xffu) << (8 * (byte % 8));
                }
            }
            n->const_bits = count;  // the element count, checked against the node's extents
            return true;
        }
        case Op::Sum:
            if (!int_of(p.get("axis"), &n->axis) || !prim_of(p.get("accumulator"), &n->accumulator))
                return (*why = "Sum needs axis and accumulator", false);
            return true;
        case Op::MaxReduce: case Op::MinReduce: case Op::ProdReduce: case Op::Argmax: case Op::Argmin:
        case Op::Softmax:
            if (!int_of(p.get("axis"), &n->axis)) return (*why = var + " needs an axis", false);
            return true;
        case Op::Count:
        case Op::Permute:
            if (!ids_of(p.get(n->op == Op::Count ? "axes" : "axes"), &n->axes)) return (*why = var + " needs axes", false);
            return true;
        case Op::Expand: {
            const Json *size = p.get("size");
            if (!int_of(p.get("axis"), &n->axis) || !size) return (*why = "Expand needs axis and size", false);
            if (!extent_of(*size, g, n, &n->size)) return (*why = "Expand size is not an extent", false);
            return true;
        }
        case Op::Reshape: {
            const Json *shape = p.get("new_shape");
            if (!shape || shape->kind != Json::Array) return (*why = "Reshape needs new_shape", false);
            for (const Json &d : shape->items) {
                int64_t e;
                if (!extent_of(d, g, n, &e)) return (*why = "Reshape new_shape holds a non-extent", false);
                n->new_shape.push_back(e);
            }
            return true;
        }
        case Op::Bitwise: {
            // BitwiseKind, snake_case (crates/chelis-numeric-core/src/bitwise.rs:8-14)
            static const char *kinds[] = {"and", "or", "xor", "shift_left", "shift_right"};
            if (p.kind != Json::String) return (*why = "Bitwise needs its kind", false);
            for (int k = 0; k < 5; ++k)
                if (p.text == kinds[k]) {
                    n->code = k;
                    return true;
                }
            return (*why = "Bitwise kind `" + p.text + "` is unknown", false);
        }
        case Op::Pad: case Op::Shrink: {
            // Vec<(RtDim, RtDim)> (dag.rs:1202-1208): [[before, after], ...] /
            // [[start, end], ...]; a shrink end may be ToEnd
            const Json *pairs = p.get(n->op == Op::Pad ? "padding" : "bounds");
            if (!pairs || pairs->kind != Json::Array) return (*why = var + " needs its bounds", false);
            for (const Json &pr : pairs->items) {
                if (pr.kind != Json::Array || pr.items.size() != 2) return (*why = var + " bounds are pairs", false);
                int64_t a = 0, b = 0;
                if (!extent_of(pr.items[0], g, n, &a)) return (*why = var + " holds a bound that is not an extent", false);
                if (n->op == Op::Shrink && pr.items[1].kind == Json::String && pr.items[1].text == "ToEnd") {
                    b = kToEnd;
                } else if (!extent_of(pr.items[1], g, n, &b)) {
                    return (*why = var + " holds a bound that is not an extent", false);
                }
                n->lo.push_back(a);
                n->hi.push_back(b);
            }
            if (n->op == Op::Pad && !scalar_of(p.get("fill"), n)) return (*why = "Pad with an unreadable fill", false);
            return true;
        }
        case Op::Stride: {
            const Json *st = p.get("strides");
            if (!st || st->kind != Json::Array) return (*why = "Stride needs its steps", false);
            for (const Json &d : st->items) {
                int64_t e = 0;
                if (!extent_of(d, g, n, &e)) return (*why = "Stride holds a step that is not an extent", false);
                n->step.push_back(e);
            }
            return true;
        }
        case Op::Compare: case Op::Logical:
            if (p.kind != Json::String) return (*why = var + " needs its kind", false);
            n->compare = p.text;
            return true;
        case Op::Gather: case Op::ScatterAdd: case Op::Scatter:
            if (!int_of(p.get("axis"), &n->axis) || !int_of(p.get("batch_rank"), &n->batch_rank))
                return (*why = var + " needs axis and batch_rank", false);
            return true;
        case Op::ScatterElements:
            if (!int_of(p.get("axis"), &n->axis)) return (*why = "ScatterElements needs an axis", false);
            return true;
        case Op::ExtremaAdjoint: {
            // ExtremaKind / ExtremaOperand (dag.rs:596-606)
            const Json *kind = p.get("kind"), *operand = p.get("operand");
            if (!kind || kind->kind != Json::String || !operand || operand->kind != Json::String ||
                (kind->text != "Max" && kind->text != "Min") || (operand->text != "Left" && operand->text != "Right"))
                return (*why = "ExtremaAdjoint needs kind Max|Min and operand Left|Right", false);
            n->code = (kind->text == "Min" ? 1 : 0) | (operand->text == "Right" ? 2 : 0);
            return true;
        }
        case Op::Cumsum: {
            const Json *dir = p.get("direction");  // ScanDirection (dag.rs:819-822)
            if (!int_of(p.get("axis"), &n->axis) || !dir || dir->kind != Json::String ||
                (dir->text != "Increasing" && dir->text != "Decreasing"))
                return (*why = "Cumsum needs axis and direction Increasing|Decreasing", false);
            n->code = dir->text == "Decreasing" ? 1 : 0;
            return true;
        }
        case Op::SplitKey: {
            const Json *branch = p.get("branch");  // KeyBranch
            if (!branch || branch->kind != Json::String || (branch->text != "Left" && branch->text != "Right"))
                return (*why = "Split needs branch Left|Right", false);
            n->code = branch->text == "Right" ? 1 : 0;
            return true;
        }
        case Op::Cast:
            if (!prim_of(p.get("new_precision"), &n->cast_to)) return (*why = "Cast needs new_precision", false);
            return true;
        case Op::NamedCast:
            return true;
        case Op::FusedElem: {
            const Json *ops = p.get("ops");
            if (!ops || ops->kind != Json::Array || ops->items.empty()) return (*why = "FusedElem needs ops", false);
            for (const Json &s : ops->items) {
                Step st;
                if (!step_op_of(s, &st)) return (*why = "FusedElem step is not a known elementwise op", false);
                n->steps.push_back(st);
            }
            return true;
        }
        default:
            return true;  // kept as read; the planner refuses what it cannot run
    }
}

}  // namespace

const char *op_name(Op op) {
    for (const OpName &o : kOps)
        if (o.op == op) return o.name;
    return "Other";
}

bool op_is_chain_step(Op op) { return op >= Op::Add && op <= Op::Round; }

const char *prim_name(Prim p) {
    for (const PrimName &q : kPrims)
        if (q.prim == p) return q.wire;
    return "Other";
}

int64_t prim_width(Prim p) {
    switch (p) {
        case Prim::F32: case Prim::Int32: return 4;
        case Prim::F64: case Prim::Int64: case Prim::Key: return 8;
        case Prim::F16: case Prim::Bf16: case Prim::Int16: return 2;
        case Prim::Int8: case Prim::Bool: return 1;
        default: return 0;
    }
}

chelis_dtype prim_dtype(Prim p) {
    switch (p) {
        case Prim::F32: return CHELIS_DTYPE_F32;
        case Prim::F64: return CHELIS_DTYPE_F64;
        case Prim::Int32: return CHELIS_DTYPE_I32;
        case Prim::Bool: return CHELIS_DTYPE_BOOL;
        case Prim::Int64: return CHELIS_DTYPE_I64;
        case Prim::Bf16: return CHELIS_DTYPE_BF16;
        case Prim::F16: return CHELIS_DTYPE_F16;
        case Prim::Int8: return CHELIS_DTYPE_I8;
        case Prim::Int16: return CHELIS_DTYPE_I16;
        case Prim::Key: return CHELIS_DTYPE_KEY;
        default: return 255;
    }
}

bool prim_is_float(Prim p) { return p == Prim::F32 || p == Prim::F64 || p == Prim::F16 || p == Prim::Bf16; }

int64_t Node::count() const {
    int64_t c = 1;
    for (int64_t d : dims) {
        if (d < 0) return -1;
        c *= d;
    }
    return c;
}

int64_t Graph::symbol(const std::string &name) {
    for (size_t s = 0; s < symbols.size(); ++s)
        if (symbols[s] == name) return (int64_t)s;
    symbols.push_back(name);
    return (int64_t)symbols.size() - 1;
}

double Node::const_value() const {
    switch (const_prec) {
        case Prim::F32: {
            float f;
            const uint32_t b = (uint32_t)const_bits;
            std::memcpy(&f, &b, 4);
            return f;
        }
        case Prim::F64: {
            double d;
            std::memcpy(&d, &const_bits, 8);
            return d;
        }
        default: return (double)(int64_t)const_bits;
    }
}

bool read_graph(const char *text, size_t n, Graph *g, std::string *error) {
    Json root;
    if (!parse_json(text, n, &root, error)) return false;
    *g = Graph{};
    const Json *nodes = root.get("nodes"), *roots = root.get("roots"), *decls = root.get("declarations");
    if (!nodes || nodes->kind != Json::Array || !roots) {
        *error = "a Dag needs nodes and roots";
        return false;
    }
    if (decls) {
        g->declarations.clear();
        write_json(*decls, &g->declarations);
    }
    for (size_t k = 0; k < nodes->items.size(); ++k) {
        const Json &j = nodes->items[k];
        Node nd;
        std::string why;
        auto bad = [&](const std::string &what) {
            *error = "node " + std::to_string(k) + ": " + what;
            return false;
        };
        if (!int_of(j.get("id"), &nd.id) || nd.id != (int64_t)k) return bad("id must equal its position");
        if (!ids_of(j.get("inputs"), &nd.inputs) || !j.get("inputs")) return bad("inputs must be node ids");
        for (int64_t in : nd.inputs)
            if (in < 0 || in >= nd.id) return bad("input " + std::to_string(in) + " does not precede the node");
        const Json *op = j.get("op");
        if (!op || !read_op(*op, g, &nd, &why)) return bad(why.empty() ? "missing op" : why);
        if (!ids_of(j.get("shape_deps"), &nd.shape_deps) || !ids_of(j.get("result_claim_deps"), &nd.claim_deps))
            return bad("shape_deps / result_claim_deps must be node ids");
        for (int64_t d : nd.shape_deps)
            if (d < 0 || d >= nd.id) return bad("shape dependency does not precede the node");
        for (int64_t d : nd.claim_deps)
            if (d < 0 || d >= nd.id) return bad("claim dependency does not precede the node");
        const Json *ty = j.get("output_type");
        if (!ty || !ty->get("dims") || ty->get("dims")->kind != Json::Array || !prim_of(ty->get("precision"), &nd.prec))
            return bad("output_type needs dims and precision");
        for (const Json &d : ty->get("dims")->items) {
            int64_t e;
            if (d.kind != Json::Object || d.fields.size() != 1 ||
                (d.fields[0].first != "Lit" && d.fields[0].first != "Named") || !extent_of(d, g, &nd, &e))
                return bad("output_type dims must be DimInfo values");
            nd.dims.push_back(e);
            std::string raw;
            write_json(d, &raw);
            nd.dims_raw.push_back(raw);
        }
        const Json *reuse = j.get("reusable_input");
        if (reuse && reuse->kind != Json::Null && !int_of(reuse, &nd.reusable)) return bad("bad reusable_input");
        if (const Json *span = j.get("span_id")) {
            if (span->kind == Json::String) {
                nd.has_span = true;
                nd.span = span->text;
            } else if (span->kind != Json::Null) {
                return bad("span_id must be a string or null");
            }
        }
        if (const Json *ms = j.get("merged_spans")) {
            if (ms->kind != Json::Array) return bad("merged_spans must be a list");
            for (const Json &s : ms->items) {
                if (s.kind != Json::String) return bad("merged_spans must hold strings");
                nd.merged_spans.push_back(s.text);
            }
        }
        const Json *owner = j.get("owner");
        if (!owner || !int_of(owner->get("decl"), &nd.owner_decl)) return bad("owner needs decl");
        const Json *act = owner->get("activation");
        if (act && act->kind != Json::Null && !int_of(act, &nd.owner_activation)) return bad("bad owner activation");
        g->nodes.push_back(std::move(nd));
    }
    if (!ids_of(roots, &g->roots)) {
        *error = "roots must be node ids";
        return false;
    }
    for (int64_t r : g->roots)
        if (r < 0 || r >= (int64_t)g->nodes.size()) {
            *error = "root " + std::to_string(r) + " is not a node";
            return false;
        }
    return true;
}

namespace {

void put_ids(std::string *o, const std::vector<int64_t> &v) {
    o->push_back('[');
    for (size_t k = 0; k < v.size(); ++k) {
        if (k) o->push_back(',');
        *o += std::to_string(v[k]);
    }
    o->push_back(']');
}

std::string fused_op_json(const Node &n) {
    std::string o = "{\"FusedElem\":{\"ops\":[";
    for (size_t s = 0; s < n.steps.size(); ++s) {
        if (s) o += ",";
        o += "{\"op\":\"";
        o += op_name(n.steps[s].op);
        o += "\",\"input_indices\":[";
        for (size_t a = 0; a < n.steps[s].args.size(); ++a) {
            if (a) o += ",";
            const int v = n.steps[s].args[a];
            o += v >= 0 ? "{\"External\":" + std::to_string(v) + "}" : "{\"PreviousStep\":" + std::to_string(-v - 1) + "}";
        }
        o += "]}";
    }
    o += "]}}";
    return o;
}

}  // namespace

std::string write_graph(const Graph &g) {
    std::string o = "{\"nodes\":[";
    for (size_t k = 0; k < g.nodes.size(); ++k) {
        const Node &n = g.nodes[k];
        if (k) o += ",";
        o += "{\"id\":" + std::to_string(n.id) + ",\"op\":";
        o += n.op == Op::FusedElem ? fused_op_json(n) : (n.raw_op.empty() ? json_quote(op_name(n.op)) : n.raw_op);
        o += ",\"inputs\":";
        put_ids(&o, n.inputs);
        o += ",\"output_type\":{\"dims\":[";
        for (size_t d = 0; d < n.dims.size(); ++d) {
            if (d) o += ",";
            if (d < n.dims_raw.size()) o += n.dims_raw[d];
            else if (extent_is_symbol(n.dims[d]))
                o += "{\"Named\":[" + json_quote(g.symbols[(size_t)extent_symbol(n.dims[d])]) + ",null]}";
            else o += "{\"Lit\":" + std::to_string(n.dims[d]) + "}";
        }
        o += "],\"precision\":" + json_quote(prim_name(n.prec)) + "}";
        o += ",\"reusable_input\":" + (n.reusable >= 0 ? std::to_string(n.reusable) : std::string("null"));
        o += ",\"span_id\":" + (n.has_span ? json_quote(n.span) : std::string("null"));
        o += ",\"merged_spans\":[";
        for (size_t s = 0; s < n.merged_spans.size(); ++s) {
            if (s) o += ",";
            o += json_quote(n.merged_spans[s]);
        }
        o += "],\"shape_deps\":";
        put_ids(&o, n.shape_deps);
        o += ",\"result_claim_deps\":";
        put_ids(&o, n.claim_deps);
        o += ",\"owner\":{\"decl\":" + std::to_string(n.owner_decl) + ",\"activation\":" +
             (n.owner_activation >= 0 ? std::to_string(n.owner_activation) : std::string("null")) + "}}";
    }
    o += "],\"roots\":";
    put_ids(&o, g.roots);
    o += ",\"declarations\":" + g.declarations + "}";
    return o;
}

}  // namespace dag
}  // namespace chelis

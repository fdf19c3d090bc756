"""Writes lowered Chelis DAGs in the reference's serde JSON shape, as fixtures
for the DAG front end (chelis_amd/csrc/dag_*.cpp).

The wire shape is the reference's `serde_json::to_string(&dag)`:
  Dag      {"nodes": [DagNode...], "roots": [id...], "declarations": [{"name", "value"}]}
  DagNode  {"id", "op", "inputs", "output_type": {"dims": [{"Lit": n} | {"Named": [name, null]}],
            "precision": "F32"},
            "reusable_input", "span_id", "merged_spans", "shape_deps", "result_claim_deps",
            "owner": {"decl": 0, "activation": null}}
  op       a unit variant as a string ("Add") or {"Variant": {fields}}
  scalar   {"dtype": "f32", "bits": "3f800000"} / {"dtype": "int64", "value": 9}
(crates/chelis-dag-core/tests/wire_behavior.rs:48,119-123;
crates/chelis-numeric-core/src/dtype_semantics/wire_codec.rs:488-512).

The node structure restates the reference's lowerings, which the Rust
compiler would run (it cannot be built here):
  matmul      Sum{L+1}(Mul(Expand{L+2}(a), Expand{L}(b)))
              (crates/chelis-dag-core/src/tier2.rs:706-857)
  softmax     decompose_softmax (tier2.rs:1098-1178)
  mean        Div(Sum, Const(extent)) (tier2.rs:1183-1245)
  layer_norm  lower_layer_norm (tier2.rs:1248-1360), expand_to_match (:629-680)
  gelu        m(x) * Phi(x) (crates/chelis-numeric-core/src/activation.rs:145-149,183-276)
  attention   spec/05-risc-primitives.md section 4.7 (scale, where(mask, s, -inf))
The MLP's reverse pass is written out as the adjoints the oracle restates
(mean, neg, sum -> expand, mul, log, softmax y * (g - sum(g * y))
crates/chelis-dag-core/src/grad.rs:2248, matmul as transposed matmuls,
dropout replay, relu adjoint), in the same lowered forms.

Run `python tests/golden/dag_builder.py` to rewrite tests/golden/dags/.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

PREC = {"f32": "F32", "f64": "F64", "bool": "Bool", "i64": "Int64", "key": "Key", "i32": "Int32", "i16": "Int16",
        "i8": "Int8", "bf16": "Bf16", "f16": "F16"}
INT_TAGS = {"i64": "int64", "i32": "int32", "i16": "int16", "i8": "int8"}
F32_LOWEST = -3.4028234663852886e38


def _f32_bits(v: float) -> str:
    return "%08x" % struct.unpack("<I", struct.pack("<f", v))[0]


def _f64_bits(v: float) -> str:
    return "%016x" % struct.unpack("<Q", struct.pack("<d", v))[0]


def _dim(d):
    """DimInfo: a literal, or a string naming an extent known only at run
    time (DimInfo::Named(name, None), crates/chelis-dag-core/src/dag.rs:276-281)."""
    return {"Named": [d, None]} if isinstance(d, str) else {"Lit": int(d)}


class Dag:
    def __init__(self, name: str = "entry"):
        self.nodes: list[dict] = []
        self.types: list[tuple[list[int], str]] = []
        self.roots: list[int] = []
        self.name = name

    # ---- raw nodes ----
    def node(self, op, inputs, dims, prec, span=None, shape_deps=()):
        nid = len(self.nodes)
        self.nodes.append({
            "id": nid, "op": op, "inputs": list(inputs),
            "output_type": {"dims": [_dim(d) for d in dims], "precision": PREC[prec]},
            "reusable_input": None, "span_id": span, "merged_spans": [], "shape_deps": list(shape_deps),
            "result_claim_deps": [], "owner": {"decl": 0, "activation": None},
        })
        self.types.append((list(dims), prec))
        return nid

    def dims(self, n):
        return self.types[n][0]

    def prec(self, n):
        return self.types[n][1]

    def json(self) -> str:
        return json.dumps({"nodes": self.nodes, "roots": self.roots,
                           "declarations": [{"name": self.name, "value": False}]}, separators=(",", ":"))

    # ---- leaves ----
    def load(self, name, dims, prec):
        return self.node({"Load": {"name": name}}, [], dims, prec, span=name)

    def const(self, value, dims, prec, shape_deps=()):
        if prec == "f32":
            v = {"dtype": "f32", "bits": _f32_bits(value)}
        elif prec == "f64":
            v = {"dtype": "f64", "bits": _f64_bits(value)}
        elif prec in INT_TAGS:
            v = {"dtype": INT_TAGS[prec], "value": int(value)}
        else:
            raise ValueError(prec)
        return self.node({"Const": {"value": v}}, [], dims, prec, shape_deps=shape_deps)

    def const_tensor(self, values, dims, prec):
        """RiscOp::ConstTensor{data} (dag.rs:1291-1293): TensorStorage's wire
        form, floats as hex bits, integers and bools as values."""
        flat = np.asarray(values).reshape(-1)
        if prec == "f32":
            data = {"dtype": "f32", "bits": [_f32_bits(float(v)) for v in flat]}
        elif prec == "f64":
            data = {"dtype": "f64", "bits": [_f64_bits(float(v)) for v in flat]}
        elif prec == "bool":
            data = {"dtype": "bool", "values": [bool(v) for v in flat]}
        else:
            data = {"dtype": INT_TAGS[prec], "values": [int(v) for v in flat]}
        return self.node({"ConstTensor": {"data": data}}, [], dims, prec)

    def drop(self, x):
        """RiscOp::Drop (dag.rs:1303-1304): a live-range close, no data moves."""
        return self.node("Drop", [x], self.dims(x), self.prec(x))

    # ---- elementwise ----
    def binary(self, op, a, b, prec=None):
        return self.node(op, [a, b], self.dims(a), prec or self.prec(a))

    def unary(self, op, a):
        return self.node(op, [a], self.dims(a), self.prec(a))

    def add(self, a, b): return self.binary("Add", a, b)
    def sub(self, a, b): return self.binary("Sub", a, b)
    def mul(self, a, b): return self.binary("Mul", a, b)
    def div(self, a, b): return self.binary("Div", a, b)
    def neg(self, a): return self.unary("Neg", a)
    def exp(self, a): return self.unary("Exp", a)
    def log(self, a): return self.unary("Log", a)
    def relu(self, a): return self.unary("Relu", a)

    def relu_adjoint(self, x, g):
        return self.node("ReluAdjoint", [x, g], self.dims(x), self.prec(x))

    def cmplt(self, a, b):
        return self.node({"Compare": "cmp_lt"}, [a, b], self.dims(a), "bool")

    def compare(self, kind, a, b):
        return self.node({"Compare": kind}, [a, b], self.dims(a), "bool")

    def where(self, c, a, b):
        return self.node("Where", [c, a, b], self.dims(a), self.prec(a))

    def logical(self, kind, a, b=None):
        """RiscOp::Logical(LogicalKind), snake_case kinds (dag.rs:553-559)."""
        return self.node({"Logical": kind}, [a] if b is None else [a, b], self.dims(a), "bool")

    def extrema_adjoint(self, kind, operand, a, b, g):
        """RiscOp::ExtremaAdjoint{kind: Max|Min, operand: Left|Right}
        (dag.rs:949-952, 596-606)."""
        return self.node({"ExtremaAdjoint": {"kind": kind, "operand": operand}}, [a, b, g], self.dims(g), self.prec(g))

    def cumsum(self, x, axis, direction="Increasing"):
        """RiscOp::Cumsum{axis, direction} (dag.rs:1408-1411); i8 / i16 scan
        into i32."""
        p = self.prec(x)
        return self.node({"Cumsum": {"axis": axis, "direction": direction}}, [x], self.dims(x),
                         "i32" if p in ("i8", "i16") else p)

    # ---- keys and draws (dag.rs:995-1060) ----
    def key_from_seed(self, seed: int):
        return self.node("KeyFromSeed", [self.const(seed, [], "i64")], [], "key")

    def split(self, key, branch):
        return self.node({"Split": {"branch": branch}}, [key], [], "key")

    def fold_in(self, key, n: int):
        return self.node("FoldIn", [key, self.const(n, [], "i64")], [], "key")

    def uniform_like(self, template, low, high, key):
        p = self.prec(template)
        return self.node("UniformLike", [template, self.const(low, [], p), self.const(high, [], p), key],
                         self.dims(template), p)

    def cast(self, x, prec):
        return self.node({"Cast": {"new_precision": PREC[prec]}}, [x], self.dims(x), prec)

    def gather(self, values, indices, axis, batch_rank=0):
        """RiscOp::Gather{axis, batch_rank} (dag.rs:1349-1356): the result is
        values[..axis] ++ indices[batch_rank..] ++ values[axis+1..]."""
        dims = self.dims(values)[:axis] + self.dims(indices)[batch_rank:] + self.dims(values)[axis + 1:]
        return self.node({"Gather": {"axis": axis, "batch_rank": batch_rank}}, [values, indices], dims,
                         self.prec(values))

    def bitwise(self, kind, a, b):
        """RiscOp::Bitwise(kind) (dag.rs:911): and, or, xor, shift_left,
        shift_right."""
        return self.node({"Bitwise": kind}, [a, b], self.dims(a), self.prec(a))

    def pad(self, x, pads, fill):
        """RiscOp::Pad{padding, fill} (dag.rs:1202-1205), literal bounds."""
        p = self.prec(x)
        if p == "f32":
            v = {"dtype": "f32", "bits": _f32_bits(fill)}
        elif p == "f64":
            v = {"dtype": "f64", "bits": _f64_bits(fill)}
        else:
            v = {"dtype": INT_TAGS[p], "value": int(fill)}
        dims = [d + a + b for d, (a, b) in zip(self.dims(x), pads)]
        padding = [[{"Lit": a}, {"Lit": b}] for a, b in pads]
        return self.node({"Pad": {"padding": padding, "fill": v}}, [x], dims, p)

    def shrink(self, x, bounds):
        """RiscOp::Shrink{bounds} (dag.rs:1206-1208): (start, end) per axis."""
        dims = [b - a for a, b in bounds]
        return self.node({"Shrink": {"bounds": [[{"Lit": a}, {"Lit": b}] for a, b in bounds]}}, [x], dims,
                         self.prec(x))

    def stride(self, x, steps):
        """RiscOp::Stride{strides} (dag.rs:1209-1211): every step-th element
        from the first."""
        dims = [-(-d // k) for d, k in zip(self.dims(x), steps)]
        return self.node({"Stride": {"strides": [{"Lit": k} for k in steps]}}, [x], dims, self.prec(x))

    def scatter(self, target, indices, updates, axis, batch_rank=0, add=False):
        """RiscOp::ScatterAdd / Scatter{axis, batch_rank} (dag.rs:1360-1384)."""
        op = "ScatterAdd" if add else "Scatter"
        return self.node({op: {"axis": axis, "batch_rank": batch_rank}}, [target, indices, updates],
                         self.dims(target), self.prec(target))

    def scatter_elements(self, data, indices, updates, axis):
        """RiscOp::ScatterElements{axis} (dag.rs:1386-1404)."""
        return self.node({"ScatterElements": {"axis": axis}}, [data, indices, updates], self.dims(data),
                         self.prec(data))

    def dropout(self, x, rate, key, replay=False):
        return self.node("DropoutReplay" if replay else "Dropout", [x, rate, key], self.dims(x), self.prec(x))

    # ---- movement ----
    def expand(self, x, axis, size, source=None, source_axis=None):
        """A literal size, or (size a run-time extent's name) the extent of
        `source`'s axis `source_axis` (default `axis`), read as
        RtDim::InputAxis{tensor: 1} with `source` as the second input
        (tier2.rs:1106-1141)."""
        d = list(self.dims(x))
        d.insert(axis, size)
        if isinstance(size, str):
            source_axis = axis if source_axis is None else source_axis
            assert source is not None and self.dims(source)[source_axis] == size
            rt = {"InputAxis": {"tensor": 1, "axis": {"Lit": source_axis}}}
            return self.node({"Expand": {"axis": axis, "size": rt}}, [x, source], d, self.prec(x))
        return self.node({"Expand": {"axis": axis, "size": {"Lit": int(size)}}}, [x], d, self.prec(x))

    def permute(self, x, axes):
        d = self.dims(x)
        return self.node({"Permute": {"axes": list(axes)}}, [x], [d[a] for a in axes], self.prec(x))

    def reshape(self, x, shape):
        return self.node({"Reshape": {"new_shape": [{"Lit": int(s)} for s in shape]}}, [x], shape, self.prec(x))

    def expand_to_match(self, x, target_dims):
        """tier2.rs:629-680: insert axes at 0 until the rank matches."""
        while len(self.dims(x)) < len(target_dims):
            missing = len(target_dims) - len(self.dims(x))
            x = self.expand(x, 0, target_dims[missing - 1])
        return x

    def scalar_like(self, value, like):
        """A constant shaped like `like` (activation.rs: every constant is
        shaped like the activation's input)."""
        return self.const(value, self.dims(like), self.prec(like))

    # ---- reductions ----
    def sum(self, x, axis):
        d = list(self.dims(x))
        del d[axis]
        acc = PREC[self.prec(x)]
        return self.node({"Sum": {"axis": axis, "accumulator": acc}}, [x], d, self.prec(x))

    def max_reduce(self, x, axis):
        d = list(self.dims(x))
        del d[axis]
        return self.node({"MaxReduce": {"axis": axis}}, [x], d, self.prec(x))

    # ---- tier 2 ----
    def mean(self, x, axis):
        s = self.sum(x, axis)
        c = self.const(float(self.dims(x)[axis]), self.dims(s), self.prec(x), shape_deps=[s])
        return self.div(s, c)

    def softmax(self, x, axis):
        n = self.dims(x)[axis]
        m = self.max_reduce(x, axis)
        me = self.expand(m, axis, n, source=x)
        shifted = self.sub(x, me)
        e = self.exp(shifted)
        s = self.sum(e, axis)
        se = self.expand(s, axis, n, source=x)
        return self.div(e, se)

    def matmul(self, a, b):
        da, db = self.dims(a), self.dims(b)
        lead = da[:-2]
        assert db[:-2] == lead, "fixtures use matching batch axes"
        L = len(lead)
        i, j, k = da[-2], da[-1], db[-1]
        assert db[-2] == j
        ae = self.expand(a, L + 2, k, source=b, source_axis=L + 1)
        be = self.expand(b, L, i, source=a, source_axis=L)
        prod = self.mul(ae, be)
        return self.sum(prod, L + 1)

    def layer_norm(self, x, gamma, beta, eps):
        dims = self.dims(x)
        axis = len(dims) - 1
        n = dims[axis]
        mean = self.mean(x, axis)
        me = self.expand(mean, axis, n)
        centered = self.sub(x, me)
        squared = self.mul(centered, centered)
        var = self.mean(squared, axis)
        ve = self.expand(var, axis, n)
        epse = self.expand_to_match(eps, dims)
        denom = self.unary("Sqrt", self.add(ve, epse))
        normed = self.div(centered, denom)
        g = self.expand_to_match(gamma, dims)
        b = self.expand_to_match(beta, dims)
        return self.add(self.mul(normed, g), b)

    def gelu(self, x):
        """activation.rs:145-149 gelu = mul(m(x), Phi(x)); guard :183-190;
        phi_graph :220-276 at f32 with PHI_F32."""
        assert self.prec(x) == "f32"
        c_, cl_, k_, s_ = 0.7071067811865476, 1.2101617485882343e-8, 1.1283791670955126, 4097.0
        # m(x)
        lowest = self.scalar_like(F32_LOWEST, x)
        below = self.cmplt(x, lowest)
        zero = self.scalar_like(0.0, x)
        nzero = self.neg(zero)
        m = self.where(below, nzero, x)
        # Phi(x)
        c = self.scalar_like(c_, x)
        cl = self.scalar_like(cl_, x)
        k = self.scalar_like(k_, x)
        s = self.scalar_like(s_, x)
        e = self.unary("Erfc", self.mul(self.neg(x), c))
        absx = self.unary("Abs", x)
        bound = self.scalar_like(64.0, x)
        inside = self.cmplt(absx, bound)
        zero2 = self.scalar_like(0.0, x)
        z = self.where(inside, x, zero2)
        a = self.neg(z)
        th = self.mul(a, c)
        ta = self.mul(s, a)
        ah = self.sub(ta, self.sub(ta, a))
        al = self.sub(a, ah)
        tc = self.mul(s, c)
        ch = self.sub(tc, self.sub(tc, c))
        cr = self.sub(c, ch)
        err = self.sub(self.mul(ah, ch), th)
        err = self.add(err, self.mul(ah, cr))
        err = self.add(err, self.mul(al, ch))
        err = self.add(err, self.mul(al, cr))
        tl = self.add(err, self.mul(a, cl))
        dens = self.exp(self.neg(self.mul(th, th)))
        corr = self.mul(self.mul(k, dens), tl)
        half = self.scalar_like(0.5, x)
        phi = self.mul(half, self.sub(e, corr))
        return self.mul(m, phi)

    def linear(self, x, w, b):
        mm = self.matmul(x, w)
        return self.add(mm, self.expand_to_match(b, self.dims(mm)))


# ---------------------------------------------------------------- programs
def softmax_program(rows, n, prec):
    g = Dag("softmax_rows")
    x = g.load("x", [rows, n], prec)
    g.roots = [g.softmax(x, 1)]
    return g


def matmul_program(m, n, k, prec):
    g = Dag("matmul")
    a = g.load("a", [m, k], prec)
    b = g.load("b", [k, n], prec)
    g.roots = [g.matmul(a, b)]
    return g


def linreg_program(n, d):
    """Config 1: r = X.w - y; grad = X^T.r / n; loss = mean(r * r) (f64)."""
    g = Dag("linreg_step")
    X = g.load("X", [n, d], "f64")
    w = g.load("w", [d], "f64")
    y = g.load("y", [n], "f64")
    wc = g.reshape(w, [d, 1])
    r2 = g.matmul(X, wc)
    r = g.sub(g.reshape(r2, [n]), y)
    Xt = g.permute(X, [1, 0])
    gs = g.matmul(Xt, g.reshape(r, [n, 1]))
    grad = g.div(g.reshape(gs, [d]), g.const(float(n), [d], "f64"))
    loss = g.mean(g.mul(r, r), 0)
    g.roots = [grad, loss]
    return g


TRANSFORMER_PARAMS = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln2_g", "ln2_b", "w1", "b1",
                      "w2", "b2")


def transformer_program(B, S, D, F, heads=None):
    """Config 4: pre-LN block, causal multi-head attention (section 4.7 with
    the mask iota(0,S)[:,None] >= iota(0,S)[None,:]), GELU FFN, f32."""
    H = heads or D // 64
    dh = D // H
    g = Dag("transformer_block")
    x = g.load("x", [B, S, D], "f32")
    p = {}
    shapes = {"ln1_g": [D], "ln1_b": [D], "wq": [D, D], "bq": [D], "wk": [D, D], "bk": [D], "wv": [D, D],
              "bv": [D], "wo": [D, D], "bo": [D], "ln2_g": [D], "ln2_b": [D], "w1": [D, F], "b1": [F], "w2": [F, D],
              "b2": [D]}
    for name in TRANSFORMER_PARAMS:
        p[name] = g.load(name, shapes[name], "f32")
    eps = g.const(1e-5, [], "f32")
    x2 = g.reshape(x, [B * S, D])
    h = g.layer_norm(x2, p["ln1_g"], p["ln1_b"], eps)

    def heads_of(t):  # [B*S, D] -> [B, H, S, dh]
        return g.permute(g.reshape(t, [B, S, H, dh]), [0, 2, 1, 3])

    q = heads_of(g.linear(h, p["wq"], p["bq"]))
    k = heads_of(g.linear(h, p["wk"], p["bk"]))
    v = heads_of(g.linear(h, p["wv"], p["bv"]))
    kt = g.permute(k, [0, 1, 3, 2])
    raw = g.matmul(q, kt)
    scale = g.const(1.0 / (dh ** 0.5), [], "f32")
    scores = g.mul(raw, g.expand_to_match(scale, g.dims(raw)))
    # causal mask [S, S]: row index >= column index, inserted over [B, H]
    start = g.const(0, [], "i64")
    end = g.const(S, [], "i64")
    iota = g.node("Iota", [start, end], [S], "i64")
    rows = g.expand(iota, 1, S)
    cols = g.expand(iota, 0, S)
    mask = g.compare("gte", rows, cols)
    maskx = g.expand_to_match(mask, g.dims(raw))
    ninf = g.const(float("-inf"), [], "f32")
    masked = g.where(maskx, scores, g.expand_to_match(ninf, g.dims(raw)))
    probs = g.softmax(masked, 3)
    o = g.matmul(probs, v)  # [B, H, S, dh]
    o2 = g.reshape(g.permute(o, [0, 2, 1, 3]), [B * S, D])
    attn = g.linear(o2, p["wo"], p["bo"])
    x1 = g.add(x2, attn)
    h2 = g.layer_norm(x1, p["ln2_g"], p["ln2_b"], eps)
    f = g.gelu(g.linear(h2, p["w1"], p["b1"]))
    y = g.add(x1, g.linear(f, p["w2"], p["b2"]))
    g.roots = [g.reshape(y, [B, S, D])]
    return g


def mlp_program(Bt, I, Hd, O, rate=0.1, lr=0.01):
    """Config 5: one SGD step of x -> relu(x W1 + b1) -> dropout(key) ->
    softmax(. W2 + b2) with cross-entropy against one-hot labels (f32)."""
    g = Dag("mlp_train_step")
    x = g.load("x", [Bt, I], "f32")
    oh = g.load("onehot", [Bt, O], "f32")
    w1 = g.load("w1", [I, Hd], "f32")
    b1 = g.load("b1", [Hd], "f32")
    w2 = g.load("w2", [Hd, O], "f32")
    b2 = g.load("b2", [O], "f32")
    key = g.load("key", [], "key")
    rate_n = g.const(rate, [], "f32")
    z1 = g.linear(x, w1, b1)
    hd = g.relu(z1)
    d = g.dropout(hd, rate_n, key)
    z2 = g.linear(d, w2, b2)
    p = g.softmax(z2, 1)
    t = g.mul(g.log(p), oh)
    nl = g.neg(g.sum(t, 1))
    loss = g.mean(nl, 0)
    # reverse pass, seeded with d loss = 1
    one = g.const(1.0, [], "f32")
    g_sum = g.div(one, g.const(float(Bt), [], "f32"))          # mean: g / extent
    g_nl = g.expand(g_sum, 0, Bt)                               # sum: expand
    g_pr = g.neg(g_nl)                                          # neg
    g_t = g.expand(g_pr, 1, O)                                  # sum over classes: expand
    g_lp = g.mul(g_t, oh)                                       # mul by the one-hot factor
    g_p = g.div(g_lp, p)                                        # log: g / x
    gy = g.mul(g_p, p)                                          # softmax adjoint
    gz2 = g.mul(p, g.sub(g_p, g.expand(g.sum(gy, 1), 1, O)))
    gb2 = g.sum(gz2, 0)
    gw2 = g.matmul(g.permute(d, [1, 0]), gz2)
    gd = g.matmul(gz2, g.permute(w2, [1, 0]))
    gh = g.dropout(gd, rate_n, key, replay=True)
    gz1 = g.relu_adjoint(z1, gh)
    gb1 = g.sum(gz1, 0)
    gw1 = g.matmul(g.permute(x, [1, 0]), gz1)
    lr_n = g.const(lr, [], "f32")

    def sgd(w, gw):
        return g.sub(w, g.mul(g.expand_to_match(lr_n, g.dims(w)), gw))

    g.roots = [loss, sgd(w1, gw1), sgd(b1, gb1), sgd(w2, gw2), sgd(b2, gb2)]
    return g


def select_program(R, N):
    """Comparison, logical and where over f32 rows: keep x where it exceeds
    the row threshold t and y is not negative, else y."""
    g = Dag("select_rows")
    x = g.load("x", [R, N], "f32")
    y = g.load("y", [R, N], "f32")
    t = g.load("t", [N], "f32")
    above = g.compare("gt", x, g.expand(t, 0, R))
    negative = g.compare("lt", y, g.const(0.0, [R, N], "f32"))
    keep = g.logical("and", above, g.logical("not", negative))
    w = g.where(keep, x, y)
    g.roots = [w, keep, g.compare("eq", w, x)]
    return g


def bitwise_program(n):
    """[05-OP-47] over i32 vectors: and, xor and both shifts by a count
    vector."""
    g = Dag("bitwise")
    a = g.load("a", [n], "i32")
    b = g.load("b", [n], "i32")
    c = g.load("c", [n], "i32")
    g.roots = [g.bitwise("and", a, b), g.bitwise("xor", a, b), g.bitwise("or", a, b),
               g.bitwise("shift_left", a, c), g.bitwise("shift_right", a, c)]
    return g


def movement_program():
    """Shrink and stride as views read by a chain, a pad of the chain's
    result, and a stride and a shrink as results."""
    g = Dag("movement")
    x = g.load("x", [512, 1000], "f32")
    s = g.shrink(x, [(10, 490), (100, 1000)])
    t = g.stride(s, [3, 2])
    y = g.binary("Add", t, g.scalar_like(1.0, t))
    g.roots = [g.pad(y, [(2, 1), (0, 5)], -1.5), g.stride(x, [2, 5]), g.shrink(x, [(500, 512), (0, 1000)])]
    return g


def scatter_program():
    """The gather's adjoint into an embedding table (duplicate ids
    accumulate by the canonical tree), a replacing scatter of rows, and an
    element-wise scatter along the last axis."""
    g = Dag("scatters")
    table = g.load("table", [5000, 64], "f32")
    ids = g.load("ids", [4096], "i64")
    grads = g.load("grads", [4096, 64], "f32")
    data = g.load("data", [512, 100], "f32")
    cols = g.load("cols", [512, 30], "i32")
    vals = g.load("vals", [512, 30], "f32")
    g.roots = [g.scatter(table, ids, grads, 0, add=True), g.scatter(table, ids, grads, 0),
               g.scatter_elements(data, cols, vals, 1)]
    return g


def literal_program():
    """A literal row added to every row of x (a ConstTensor read through an
    Expand), a literal i32 tensor as a result, and a Drop of an input."""
    g = Dag("literals")
    x = g.load("x", [256, 1000], "f32")
    y = g.load("y", [3, 4], "i32")
    row = g.const_tensor(np.float32(np.arange(1000)) * np.float32(0.37) - np.float32(100.5), [1000], "f32")
    grid = g.const_tensor(np.arange(12).reshape(3, 4) * 7 - 40, [3, 4], "i32")
    out = g.binary("Add", x, g.expand(row, 0, 256))
    total = g.bitwise("xor", y, grid)
    g.drop(y)
    g.roots = [out, grid, total]
    return g


def cast_program(n):
    """Checked casts of an f64 vector: rounded to i32, and narrowed to f32
    and bf16."""
    g = Dag("casts")
    x = g.load("x", [n], "f64")
    g.roots = [g.cast(g.unary("Round", x), "i32"), g.cast(x, "f32"), g.cast(x, "bf16")]
    return g


def integer_program(n, prec="i64"):
    """Checked integer arithmetic: floor and truncating division, the
    remainder, max_elem and sub, none of them in a fused chain."""
    g = Dag("integer_ops")
    a = g.load("a", [n], prec)
    b = g.load("b", [n], prec)
    q = g.binary("FloorDiv", a, b)
    r = g.binary("Mod", a, b)
    m = g.binary("MaxElem", q, r)
    g.roots = [q, r, g.binary("Sub", a, m), g.binary("TruncDiv", a, b)]
    return g


def gather_program(V, D, B, T):
    """Row gather (an embedding lookup) and a batched gather of one column
    per row (a label's logit)."""
    g = Dag("gathers")
    table = g.load("table", [V, D], "f32")
    ids = g.load("ids", [B], "i64")
    logits = g.load("logits", [B, T], "f32")
    labels = g.load("labels", [B, 1], "i64")
    g.roots = [g.gather(table, ids, 0), g.gather(logits, labels, 1, batch_rank=1)]
    return g


def draws_program(R, N, seed=1234):
    """A uniform draw and a dropout whose keys the plan derives from a
    literal seed (key_from_seed, split, fold_in)."""
    g = Dag("draws")
    x = g.load("x", [R, N], "f32")
    k0 = g.key_from_seed(seed)
    u = g.uniform_like(x, -1.0, 2.0, g.fold_in(g.split(k0, "Left"), 7))
    d = g.dropout(x, g.const(0.1, [], "f32"), g.split(k0, "Right"))
    g.roots = [u, d]
    return g


def scan_program(R, N):
    """Ordered scans: running sums along rows and, from the end, along
    columns (f32), and an i64 running total."""
    g = Dag("scans")
    x = g.load("x", [R, N], "f32")
    c = g.load("c", [R], "i64")
    g.roots = [g.cumsum(x, 1), g.cumsum(x, 0, "Decreasing"), g.cumsum(c, 0)]
    return g


def extrema_adjoint_program(R, N):
    g = Dag("extrema_adjoints")
    a = g.load("a", [R, N], "f32")
    b = g.load("b", [R, N], "f32")
    c = g.load("g", [R, N], "f32")
    g.roots = [g.extrema_adjoint("Max", "Left", a, b, c), g.extrema_adjoint("Max", "Right", a, b, c),
               g.extrema_adjoint("Min", "Left", a, b, c)]
    return g


FIXTURES = {
    "softmax_f32_16384x1024": lambda: softmax_program(16384, 1024, "f32"),
    "softmax_f64_4096x4096": lambda: softmax_program(4096, 4096, "f64"),
    # run-time extents: the row count, and both extents (the softmax axis
    # then reaches its expands as InputAxis reads of x, tier2.rs:1106-1114)
    "softmax_f32_rows_x1024": lambda: softmax_program("rows", 1024, "f32"),
    "softmax_f32_rows_x_cols": lambda: softmax_program("rows", "cols", "f32"),
    "gemm_f32_4096": lambda: matmul_program(4096, 4096, 4096, "f32"),
    "gemm_f64_4096": lambda: matmul_program(4096, 4096, 4096, "f64"),
    "skinny_f64_8192x64x4096": lambda: matmul_program(8192, 64, 4096, "f64"),
    "gemv_f64_8192": lambda: matmul_program(8192, 1, 8192, "f64"),
    "linreg_step_8192x32": lambda: linreg_program(8192, 32),
    "transformer_block_b8_s512_d1024": lambda: transformer_program(8, 512, 1024, 4096),
    "mlp_train_step_1024x784x512x10": lambda: mlp_program(1024, 784, 512, 10),
    "select_rows_f32_4096x1024": lambda: select_program(4096, 1024),
    "casts_f64_65536": lambda: cast_program(65536),
    "integer_ops_i64_65536": lambda: integer_program(65536),
    "gathers_50000x64_4096x10": lambda: gather_program(50000, 64, 4096, 10),
    "draws_f32_1024x512": lambda: draws_program(1024, 512),
    "extrema_adjoints_f32_4096x1024": lambda: extrema_adjoint_program(4096, 1024),
    "scans_f32_512x1024": lambda: scan_program(512, 1024),
    "bitwise_i32_65536": lambda: bitwise_program(65536),
    "movement_f32_512x1000": movement_program,
    "scatters_5000x64_4096": scatter_program,
    "literals_f32_256x1000": literal_program,
}

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dags")


def main():
    os.makedirs(OUT, exist_ok=True)
    for name, make in FIXTURES.items():
        with open(os.path.join(OUT, name + ".json"), "w") as fh:
            fh.write(make().json() + "\n")


if __name__ == "__main__":
    main()

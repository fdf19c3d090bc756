"""The DAG front end on the host (no GPU): the reference's wire form read
and written back byte for byte, fuse.rs's chain rules, the region plans of
the configuration programs, unsupported ops named, and the codegen surface
(its source compiles against the library's headers)."""
import ctypes
import json
import os
import subprocess
import sys
import tempfile

import pytest

import chelis_amd as C

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import dag_builder as DB  # noqa: E402

DAGS = os.path.join(HERE, "golden", "dags")

# crates/chelis-dag-core/tests/wire_behavior.rs:119-123: the golden Dag JSON
WIRE_GOLDEN = (
    '{"nodes":[{"id":0,"op":{"Load":{"name":"grads.1"}},"inputs":[],"output_type":{"dims":[],"precision":"Int64"},'
    '"reusable_input":null,"span_id":"x","merged_spans":[],"shape_deps":[],"result_claim_deps":[],'
    '"owner":{"decl":0,"activation":null}},{"id":1,"op":{"Const":{"value":{"dtype":"int64","value":9007199254740993}}},'
    '"inputs":[],"output_type":{"dims":[],"precision":"Int64"},"reusable_input":null,"span_id":"c","merged_spans":[],'
    '"shape_deps":[],"result_claim_deps":[],"owner":{"decl":0,"activation":null}}],"roots":[1,0],'
    '"declarations":[{"name":"fixture","value":false}]}')

# wire_behavior.rs:48 (one node) and :69 (the form without the optional lists)
NODE_GOLDEN = ('{"id":1,"op":"Neg","inputs":[0],"output_type":{"dims":[{"Lit":3}],"precision":"F32"},'
               '"reusable_input":0,"span_id":"op","merged_spans":["extra"],"shape_deps":[0],"result_claim_deps":[],'
               '"owner":{"decl":0,"activation":null}}')
OLD_NODE = ('{"id":0,"op":"Neg","inputs":[],"output_type":{"dims":[],"precision":"F32"},"reusable_input":null,'
            '"owner":{"decl":0,"activation":null}}')


def test_wire_golden_round_trips_byte_for_byte():
    assert C.dag_fuse(WIRE_GOLDEN) == WIRE_GOLDEN


def test_node_golden_round_trips_and_old_form_reads():
    load = ('{"id":0,"op":{"Load":{"name":"x"}},"inputs":[],"output_type":{"dims":[{"Lit":3}],"precision":"F32"},'
            '"reusable_input":null,"span_id":null,"merged_spans":[],"shape_deps":[],"result_claim_deps":[],'
            '"owner":{"decl":0,"activation":null}}')
    text = '{"nodes":[' + load + ',' + NODE_GOLDEN + '],"roots":[1],"declarations":[]}'
    assert C.dag_fuse(text) == text
    old = '{"nodes":[' + OLD_NODE.replace('"inputs":[]', '"inputs":[]') + '],"roots":[0],"declarations":[]}'
    back = json.loads(C.dag_fuse(old))
    assert back["nodes"][0]["span_id"] is None and back["nodes"][0]["shape_deps"] == []


@pytest.mark.parametrize("bad,what", [
    ('{"nodes":[{"id":1,"op":"Neg","inputs":[],"output_type":{"dims":[],"precision":"F32"},'
     '"reusable_input":null,"owner":{"decl":0,"activation":null}}],"roots":[0],"declarations":[]}', "id must equal"),
    ('{"nodes":[{"id":0,"op":"Neg","inputs":[0],"output_type":{"dims":[],"precision":"F32"},'
     '"reusable_input":null,"owner":{"decl":0,"activation":null}}],"roots":[0],"declarations":[]}', "does not precede"),
    ('{"nodes":[{"id":0,"op":"Neg","inputs":[],"output_type":{"dims":[],"precision":"F32"},'
     '"reusable_input":null}],"roots":[0],"declarations":[]}', "owner"),
    ('{"nodes":[],"roots":[3],"declarations":[]}', "root 3"),
    ('{"nodes":[', "byte"),
])
def test_malformed_dags_are_refused_with_the_reason(bad, what):
    with pytest.raises(C.ChelisError, match=what):
        C.dag_fuse(bad)


def fused(g):
    return json.loads(C.dag_fuse(g.json()))


def ops(d):
    return [n["op"] if isinstance(n["op"], str) else next(iter(n["op"])) for n in d["nodes"]]


def test_fuse_softmax_is_the_four_kernel_form():
    """decompose_softmax fused by fuse.rs: the sub and exp chain (exp has two
    readers, so it ends there), a lone Div stays a Div."""
    d = fused(DB.softmax_program(4, 8, "f32"))
    assert ops(d) == ["Load", "MaxReduce", "Expand", "FusedElem", "Sum", "Expand", "Div"]
    fe = d["nodes"][3]["op"]["FusedElem"]["ops"]
    assert [s["op"] for s in fe] == ["Sub", "Exp"]
    assert fe[0]["input_indices"] == [{"External": 0}, {"External": 1}]
    assert fe[1]["input_indices"] == [{"PreviousStep": 0}]
    assert d["nodes"][3]["inputs"] == [0, 2]


def test_fuse_layer_norm_tail_is_one_five_step_chain():
    g = DB.Dag("ln")
    x = g.load("x", [4, 16], "f32")
    gm, bt = g.load("g", [16], "f32"), g.load("b", [16], "f32")
    g.roots = [g.layer_norm(x, gm, bt, g.const(1e-5, [], "f32"))]
    d = fused(g)
    chains = [n["op"]["FusedElem"]["ops"] for n in d["nodes"] if not isinstance(n["op"], str) and "FusedElem" in n["op"]]
    assert [[s["op"] for s in c] for c in chains] == [["Add", "Sqrt", "Div", "Mul", "Add"]]
    # the centered value has three readers (mul twice, div): it stays a Sub
    assert ops(d).count("Sub") == 1


def test_fuse_rules_single_consumer_owner_and_length():
    g = DB.Dag("rules")
    x = g.load("x", [8], "f32")
    a = g.neg(x)            # one reader: chains into exp
    b = g.exp(a)            # two readers: the chain ends here
    c = g.add(b, b)         # alone: a one-node chain stays a plain Add
    e = g.log(b)
    f = g.unary("Sqrt", e)  # log -> sqrt chains
    g.roots = [c, f]
    d = fused(g)
    assert ops(d) == ["Load", "FusedElem", "Add", "FusedElem"]
    assert [s["op"] for s in d["nodes"][1]["op"]["FusedElem"]["ops"]] == ["Neg", "Exp"]
    assert [s["op"] for s in d["nodes"][3]["op"]["FusedElem"]["ops"]] == ["Log", "Sqrt"]
    assert d["roots"] == [2, 3]


def plan(name_or_text):
    text = name_or_text if name_or_text.startswith("{") else open(os.path.join(DAGS, name_or_text + ".json")).read()
    return C.DagProgram(text)


def kinds(p):
    return [line.split()[1] for line in p.describe().strip().splitlines()]


def with_roots_reversed(name):
    """The fixture with its roots in reverse order: the same values, but not
    the lowered program the whole-program regions recognize."""
    d = json.load(open(os.path.join(DAGS, name + ".json")))
    d["roots"] = d["roots"][::-1]
    return json.dumps(d, separators=(",", ":"))


def test_plans_of_the_configuration_programs():
    assert kinds(plan("softmax_f32_16384x1024")) == ["softmax"]
    assert kinds(plan("gemm_f32_4096")) == ["matmul"]
    # the whole linear-regression step: the fused program (two launches)
    assert kinds(plan("linreg_step_8192x32")) == ["linreg_step"]
    assert kinds(plan(with_roots_reversed("linreg_step_8192x32"))) == ["matmul", "chain", "matmul", "chain", "reduce",
                                                                        "chain"]
    t = plan("transformer_block_b8_s512_d1024")
    # Q, K and V as one batched product; the scores product, causal softmax
    # and P.V fold into one attention region
    assert kinds(t) == ["layer_norm", "matmul_group", "attention", "matmul", "layer_norm", "matmul", "matmul"]
    desc = t.describe().splitlines()
    assert "causal" in desc[2] and "permuted" in desc[2]
    assert "bias gelu" in desc[5] and "bias residual" in desc[6] and "-> output 0" in desc[6]
    # the slot plan reuses ranges: [4096, 1024] f32 for the layer norms and
    # attention, the Q/K/V block (three of them back to back) then the
    # output projection, and the [4096, 4096] FFN hidden layer; no scores
    n_const = sum(1 for n in json.load(open(os.path.join(DAGS, "transformer_block_b8_s512_d1024.json")))["nodes"]
                  if isinstance(n["op"], dict) and "Const" in n["op"])
    assert t.peak_device_bytes == 4 * 8 * 512 * 1024 * 4 + 8 * 512 * 4096 * 4 + 8 * n_const
    assert kinds(plan("mlp_train_step_1024x784x512x10")) == ["mlp_step"]
    m = plan(with_roots_reversed("mlp_train_step_1024x784x512x10"))
    k = kinds(m)
    assert k.count("matmul") == 5 and k.count("softmax") == 1 and k.count("softmax_adjoint") == 1
    assert k.count("dropout") == 2 and k.count("relu") == 1 and k.count("relu_adjoint") == 1
    # output labels are the reference's output specs: "root<index>"
    # (crates/chelis-backend-hip/src/emit.rs:5923-5930)
    assert [o[0] for o in m.outputs] == ["root0", "root1", "root2", "root3", "root4"]
    assert [o[1] for o in m.outputs] == [(10,), (512, 10), (512,), (784, 512), ()]
    assert [i[0] for i in m.inputs] == ["x", "onehot", "w1", "b1", "w2", "b2", "key"]


def test_a_pattern_with_an_outside_reader_is_not_taken():
    """A softmax whose exp is also a root must not hide the exp inside one
    kernel: the plan falls back to the generic regions."""
    g = DB.Dag("shared")
    x = g.load("x", [4, 8], "f32")
    sm = g.softmax(x, 1)
    e = g.nodes[sm]["inputs"][0]
    g.roots = [sm, e]
    assert "softmax" not in kinds(plan(g.json()))


def test_unsupported_ops_are_named():
    g = DB.Dag("pow")
    x = g.load("x", [4], "f32")
    g.roots = [g.binary("Pow", x, x)]
    with pytest.raises(C.ChelisError, match="Pow has no device chain step"):
        plan(g.json())


def test_codegen_surface_and_its_source_compiles():
    text = open(os.path.join(DAGS, "linreg_step_8192x32.json")).read()
    r = C.CodegenResult(text, "linreg_step_dag")
    assert r.input_labels == ["X", "w", "y"] and r.output_labels == ["root0", "root1"]
    assert r.symbolic_dims == [] and r.peak_device_bytes_estimate == plan("linreg_step_8192x32").peak_device_bytes
    assert "-lchelis_hip" in r.link_flags
    assert "extern \"C\" void linreg_step_dag_device(" in r.c_source
    assert "linreg_step_dag(chelis_tensor **inputs" in r.h_header
    with pytest.raises(C.ChelisError, match="C identifier"):
        C.CodegenResult(text, "not an identifier")
    with tempfile.TemporaryDirectory() as tmp:
        src = os.path.join(tmp, "gen.cpp")
        with open(src, "w") as fh:
            fh.write(r.c_source)
        lib = os.path.join(tmp, "libgen.so")
        cmd = ["g++", "-shared", "-fPIC", *r.compile_flags, src, "-o", lib, *r.link_flags]
        out = subprocess.run(cmd, capture_output=True, text=True)
        assert out.returncode == 0, out.stderr[-3000:]
        syms = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True).stdout
        assert " linreg_step_dag_device" in syms and " linreg_step_dag\n" in syms


# ---------------------------------------------------------------- run-time extents
def node(nid, op, inputs, dims, prec="F32", claims=(), span=None):
    """One DagNode in the wire form; dims are DimInfo values."""
    return {"id": nid, "op": op, "inputs": list(inputs), "output_type": {"dims": list(dims), "precision": prec},
            "reusable_input": None, "span_id": span, "merged_spans": [], "shape_deps": [],
            "result_claim_deps": list(claims), "owner": {"decl": 0, "activation": None}}


def dag(nodes, roots):
    return json.dumps({"nodes": nodes, "roots": roots, "declarations": [{"name": "t", "value": False}]},
                      separators=(",", ":"))


LIT = lambda n: {"Lit": n}  # noqa: E731
NAMED = lambda s, n=None: {"Named": [s, n]}  # noqa: E731


def fake_packet(shape, dtype=0, width=4):
    """A packet with a dummy device address: the binding and shape queries
    read only metadata, so no device is touched."""
    n = len(shape)
    sh = (ctypes.c_int64 * max(1, n))(*shape)
    st = (ctypes.c_int64 * max(1, n))()
    acc = 1
    for a in reversed(range(n)):
        st[a] = acc
        acc *= max(1, shape[a])
    t = C.GpuTensor()
    t.data, t.shape, t.strides, t.rank, t.dtype = 0x10000, sh, st, n, dtype
    t.count = 1
    for e in shape:
        t.count *= e
    t.byte_capacity = max(1, t.count) * width
    t._keep = (sh, st)
    return t


class Fake:
    def __init__(self, shape, dtype=0, width=4):
        self.t = fake_packet(shape, dtype, width)
        self.packet = ctypes.pointer(self.t)


def test_named_extents_round_trip_byte_for_byte():
    """DimInfo::Named with and without a value, an RtDim::Sym reshape target
    and an InputAxis expand are written back exactly as read."""
    text = dag([node(0, {"Load": {"name": "x"}}, [], [NAMED("rows"), NAMED("n", 4)], span="x"),
                node(1, {"MaxReduce": {"axis": 1}}, [0], [NAMED("rows")]),
                node(2, {"Expand": {"axis": 1, "size": {"InputAxis": {"tensor": 1, "axis": {"Lit": 1}}}}}, [1, 0],
                     [NAMED("rows"), NAMED("n", 4)]),
                node(3, {"Reshape": {"new_shape": [{"Sym": "rows"}, {"Lit": 4}]}}, [2], [NAMED("rows"), LIT(4)])],
               [3])
    assert C.dag_fuse(text) == text
    # the fused form keeps a chain's run-time extents too
    sm = open(os.path.join(DAGS, "softmax_f32_rows_x_cols.json")).read().strip()
    fe = [n for n in json.loads(C.dag_fuse(sm))["nodes"] if isinstance(n["op"], dict) and "FusedElem" in n["op"]]
    assert fe and fe[0]["output_type"]["dims"] == [NAMED("rows"), NAMED("cols")]
    assert "Lit\":-1" not in C.dag_fuse(sm)


def test_softmax_with_run_time_extents_binds_them_from_its_input():
    """tier2.rs:2964 softmax_accepts_symbolic_axis_extent: the expands read
    the softmax axis from x; the plan is still the one softmax region and
    binds both extents from the input packet at each call."""
    p = C.DagProgram(open(os.path.join(DAGS, "softmax_f32_rows_x_cols.json")).read())
    assert kinds(p) == ["softmax"]
    assert p.symbolic_dims == ["rows", "cols"]
    assert p.inputs == [("x", (-1, -1), 0)] and p.outputs == [("root0", (-1, -1), 0)]
    for shape in [(3, 5), (4096, 1024)]:
        assert p.output_shapes([Fake(shape)]) == [shape]
    with pytest.raises(C.ChelisError, match="rank"):
        p.output_shapes([Fake((3, 5, 1))])
    r = C.CodegenResult(open(os.path.join(DAGS, "softmax_f32_rows_x_cols.json")).read(), "softmax_rows")
    assert r.symbolic_dims == ["rows", "cols"]
    assert "chelis_device_metadata rows = input_view_0->shape[0];" in r.c_source
    assert "chelis_output_shape_0[2] = { rows, cols };" in r.c_source


def test_a_slot_sized_by_a_run_time_extent_has_a_symbolic_peak():
    g = DB.Dag("sym")
    x = g.load("x", ["rows", 1024], "f32")
    sm = g.softmax(x, 1)
    g.roots = [g.add(sm, sm)]
    p = plan(g.json())
    assert kinds(p) == ["softmax", "chain"]
    assert p.peak_device_bytes == -1
    assert p.peak_device_bytes_at(rows=3) == 3 * 4096
    assert p.peak_device_bytes_at(rows=5) == 5 * 4096
    r = C.CodegenResult(g.json(), "sym")
    assert r.peak_device_bytes_formula == "4096*rows" and r.peak_device_bytes_estimate is None
    # a size expression whose coefficient is not a multiple of 256 is rounded
    g2 = DB.Dag("odd")
    y = g2.load("y", ["n", 3], "f32")
    s2 = g2.softmax(y, 1)
    g2.roots = [g2.add(s2, s2)]
    p2 = plan(g2.json())
    assert C.CodegenResult(g2.json(), "odd").peak_device_bytes_formula == "round_up(12*n, 256)"
    assert p2.peak_device_bytes_at(n=1) == 256 and p2.peak_device_bytes_at(n=22) == 512


def test_agreeing_declarations_of_one_extent_are_checked():
    g = DB.Dag("two")
    x, y = g.load("x", ["n", 4], "f32"), g.load("y", ["n", 4], "f32")
    g.roots = [g.add(g.exp(x), y)]
    p = plan(g.json())
    assert p.symbolic_dims == ["n"]
    assert p.output_shapes([Fake((3, 4)), Fake((3, 4))]) == [(3, 4)]
    with pytest.raises(C.ChelisError, match=r"symbolic dim `n` mismatch: y\[0\]=5 but n=3"):
        p.output_shapes([Fake((3, 4)), Fake((5, 4))])
    r = C.CodegenResult(g.json(), "two")
    assert "symbolic dim `n` mismatch: y[0]=%lld but n=%lld" in r.c_source


def test_extents_this_build_cannot_bind_are_refused_never_written_as_literals():
    read_from_node = dag([node(0, {"Load": {"name": "x"}}, [], [LIT(4)], span="x"),
                          node(1, {"Load": {"name": "k"}}, [], [], prec="Int64"),
                          node(2, {"Expand": {"axis": 0, "size": {"Node": 1}}}, [0, 1], [NAMED("m"), LIT(4)])],
                         [2])
    assert C.dag_fuse(read_from_node) == read_from_node
    with pytest.raises(C.ChelisError, match="a bound read from a node value is a run-time extent"):
        plan(read_from_node)
    with pytest.raises(C.ChelisError, match="run-time extent"):
        C.CodegenResult(read_from_node, "f")
    undeclared = dag([node(0, {"Load": {"name": "x"}}, [], [LIT(4)], span="x"),
                      node(1, {"Reshape": {"new_shape": [{"Sym": "k"}, {"Lit": 2}]}}, [0], [NAMED("k"), LIT(2)])],
                     [1])
    with pytest.raises(C.ChelisError, match="run-time extent `k` is not declared by any input"):
        plan(undeclared)


def test_output_specs_follow_the_reference():
    """emit.rs:5881-5933: one input slot per Load name, Store nodes first
    under their names, then each root once as root<index>."""
    text = dag([node(0, {"Load": {"name": "x"}}, [], [LIT(4)], span="x"),
                node(1, {"Load": {"name": "x"}}, [], [LIT(4)], span="x"),
                node(2, "Neg", [0], [LIT(4)]),
                node(3, "Exp", [1], [LIT(4)]),
                node(4, {"Store": {"name": "grads.1"}}, [3], [LIT(4)])],
               [2, 2, 3])
    p = plan(text)
    assert [i[0] for i in p.inputs] == ["x"]
    assert [o[0] for o in p.outputs] == ["grads.1", "root0", "root2"]


def test_extent_witness_requirements_are_checked_before_a_run():
    witness = {"ExtentWitness": {"site": "Caller", "parameter": "x", "axis": {"Lit": 0},
                                 "requirements": [{"dtype": "int64", "value": 4}], "claims": []}}
    text = dag([node(0, {"Load": {"name": "x"}}, [], [NAMED("n"), LIT(2)], span="x"),
                node(1, witness, [], [], prec="Int64"),
                node(2, "Neg", [0], [NAMED("n"), LIT(2)])],
               [2])
    p = plan(text)
    assert p.output_shapes([Fake((4, 2))]) == [(4, 2)]
    with pytest.raises(C.ChelisError, match="extent `x` axis 0: claimed = 4, got 5"):
        p.output_shapes([Fake((5, 2))])


# ---------------------------------------------------------------- fuse's claim barrier
LITERAL_CLAIM = {"ExtentWitness": {"site": "LiteralResultClaim", "parameter": "", "axis": {"Lit": 0},
                                   "requirements": [{"dtype": "int64", "value": 4}], "claims": []}}


def test_a_claimed_producer_neither_starts_nor_joins_a_chain():
    """fuse.rs:147-161,183 with axis_sources.rs:3693-3753. Without the
    barrier Neg -> Exp is one two-step chain; with a result claim on Neg it
    cannot start one, and Exp alone is not a chain, so the DAG is unchanged."""
    free = dag([node(0, {"Load": {"name": "x"}}, [], [LIT(4)], span="x"),
                node(1, LITERAL_CLAIM, [], [], prec="Int64"),
                node(2, "Neg", [0], [LIT(4)]),
                node(3, "Exp", [2], [LIT(4)])], [3])
    assert ops(json.loads(C.dag_fuse(free))) == ["Load", "ExtentWitness", "FusedElem"]
    claimed = json.loads(free)
    claimed["nodes"][2]["result_claim_deps"] = [1]
    text = json.dumps(claimed, separators=(",", ":"))
    assert C.dag_fuse(text) == text
    # the claim on the chain's end stops the extension into it
    end = json.loads(free)
    end["nodes"][3]["result_claim_deps"] = [1]
    text = json.dumps(end, separators=(",", ":"))
    assert C.dag_fuse(text) == text


def test_the_claim_barrier_follows_copies_and_casts():
    """A Copy that owns a claim protects its input (the transitive walk,
    axis_sources.rs:3713-3731): Exp cannot join Neg's chain."""
    d = {"nodes": [node(0, {"Load": {"name": "x"}}, [], [LIT(4)], span="x"),
                   node(1, LITERAL_CLAIM, [], [], prec="Int64"),
                   node(2, "Neg", [0], [LIT(4)]),
                   node(3, "Exp", [2], [LIT(4)]),
                   node(4, "Copy", [3], [LIT(4)], claims=[1])],
         "roots": [4], "declarations": []}
    text = json.dumps(d, separators=(",", ":"))
    assert C.dag_fuse(text) == text
    d["nodes"][4]["result_claim_deps"] = []  # no claim: Neg -> Exp fuse
    assert ops(json.loads(C.dag_fuse(json.dumps(d)))) == ["Load", "ExtentWitness", "FusedElem", "Copy"]


def test_a_division_under_an_activation_keeps_its_own_kernel():
    """dag.rs:2555-2556,2864-2880: every Div may fail its check, so under an
    activation it is not fused; Exp -> Log under the same activation is."""
    d = {"nodes": [node(0, {"Load": {"name": "on"}}, [], [], prec="Bool", span="on"),
                   node(1, {"Load": {"name": "x"}}, [], [LIT(4)], span="x"),
                   node(2, "Exp", [1], [LIT(4)]),
                   node(3, "Div", [2, 2], [LIT(4)]),
                   node(4, "Log", [3], [LIT(4)]),
                   node(5, "Sqrt", [4], [LIT(4)])],
         "roots": [5], "declarations": []}
    for n in d["nodes"][2:]:
        n["owner"]["activation"] = 0
    assert ops(json.loads(C.dag_fuse(json.dumps(d)))) == ["Load", "Load", "Exp", "Div", "FusedElem"]


# ---------------------------------------------------------------- generated entry traps
def _generated(tmp, name="linreg_step_8192x32", func="gen"):
    r = C.CodegenResult(open(os.path.join(DAGS, name + ".json")).read(), func)
    src = os.path.join(tmp, "gen.cpp")
    with open(src, "w") as fh:
        fh.write(r.c_source)
    lib = os.path.join(tmp, "libgen.so")
    out = subprocess.run(["g++", "-shared", "-fPIC", *r.compile_flags, src, "-o", lib, *r.link_flags],
                         capture_output=True, text=True)
    assert out.returncode == 0, out.stderr[-3000:]
    return lib


CHILD = r"""
import ctypes, sys
lib = ctypes.CDLL(sys.argv[1])
case = sys.argv[2]
arr = (ctypes.c_void_p * 4)()
if case == "device_arity":
    lib.gen_device(arr, 2, arr, 2)
elif case == "device_outputs":
    lib.gen_device(arr, 3, arr, 5)
elif case == "device_null":
    lib.gen_device(None, 3, arr, 2)
elif case == "host_arity":
    lib.gen(arr, 1, arr, 2)
elif case == "host_null":
    lib.gen(arr, 3, None, 2)
"""


@pytest.mark.parametrize("case,status,text", [
    ("device_arity", -6, "gen_device: expected 3 inputs, got 2"),
    ("device_outputs", -6, "gen_device: expected 2 outputs, got 5"),
    ("device_null", 1, "numeric trap: domain in entry at i64"),
    ("host_arity", -6, "gen: expected 3 inputs, got 1"),
    ("host_null", 1, "numeric trap: domain in entry at i64"),
])
def test_generated_entries_trap_as_the_reference_does(case, status, text):
    """emit.rs:676-695,857-876: a count mismatch prints and aborts; null
    arrays are a `domain` numeric trap (exit status 1). Both are checked
    before any HIP call, so they run without a device."""
    with tempfile.TemporaryDirectory() as tmp:
        lib = _generated(tmp)
        r = subprocess.run([sys.executable, "-c", CHILD, lib, case], capture_output=True, text=True, timeout=120)
    assert r.returncode == status, (r.returncode, r.stderr[-2000:])
    assert text in r.stderr


# ---------------------------------------------------------------- build-side surface
def blas_nodes(text):
    return [n for n in json.loads(text)["nodes"] if isinstance(n["op"], dict) and "BlasMatmul" in n["op"]]


def test_prepare_selects_blas_matmul_and_is_idempotent():
    """lib.rs:173-227 over specialize.rs:150-226: a lowered matmul becomes one
    BlasMatmul node (its Mul and Expands dropped); applying it again changes
    nothing; the plan is the same launches."""
    text = DB.matmul_program(64, 48, 32, "f32").json()
    p = C.prepare_dag_for_codegen(text)
    assert ops(json.loads(p)) == ["Load", "Load", "BlasMatmul"]
    (bm,) = blas_nodes(p)
    assert bm["op"]["BlasMatmul"] == {"batch_dims": [], "m": {"Concrete": 64}, "n": {"Concrete": 48},
                                      "k": {"Concrete": 32}, "accumulator": "F32"}
    assert bm["inputs"] == [0, 1]
    assert C.prepare_dag_for_codegen(p) == p
    assert kinds(plan(p)) == kinds(plan(text)) == ["matmul"]


def test_prepare_leaves_transposed_operands_and_claimed_regions():
    """specialize.rs:795-900: an operand read through a Permute has no
    contiguous matrix slices, so the MLP's gradient products stay lowered
    while its two forward products are selected; a matched region that owns
    a result claim is not rewritten."""
    mlp = open(os.path.join(DAGS, "mlp_train_step_1024x784x512x10.json")).read()
    p = C.prepare_dag_for_codegen(mlp)
    assert [(b["op"]["BlasMatmul"]["m"], b["op"]["BlasMatmul"]["n"], b["op"]["BlasMatmul"]["k"])
            for b in blas_nodes(p)] == [({"Concrete": 1024}, {"Concrete": 512}, {"Concrete": 784}),
                                        ({"Concrete": 1024}, {"Concrete": 10}, {"Concrete": 512})]
    assert kinds(plan(p)) == kinds(plan(mlp))
    d = json.loads(DB.matmul_program(8, 4, 2, "f64").json())
    d["nodes"].append(node(len(d["nodes"]), LITERAL_CLAIM, [], [], prec="Int64"))
    d["nodes"][-2]["result_claim_deps"] = [len(d["nodes"]) - 1]
    d["nodes"][-1], d["nodes"][-2] = d["nodes"][-2], d["nodes"][-1]  # the witness precedes its owner
    d["nodes"][-2]["id"], d["nodes"][-1]["id"] = len(d["nodes"]) - 2, len(d["nodes"]) - 1
    d["nodes"][-1]["result_claim_deps"] = [len(d["nodes"]) - 2]
    d["roots"] = [len(d["nodes"]) - 1]
    text = json.dumps(d, separators=(",", ":"))
    assert blas_nodes(C.prepare_dag_for_codegen(text)) == []


def test_prepare_keeps_run_time_extents_as_symbols():
    g = DB.Dag("sym")
    a, b = g.load("a", ["m", 16], "f32"), g.load("b", [16, 8], "f32")
    g.roots = [g.matmul(a, b)]
    (bm,) = blas_nodes(C.prepare_dag_for_codegen(g.json()))
    assert bm["op"]["BlasMatmul"]["m"] == {"Sym": "m"} and bm["output_type"]["dims"][0] == NAMED("m")


def test_tensor_capable_prims_and_runtime_dir():
    # lib.rs:10-18: F32, F64, Bool, Bf16, F16, Int32, Int64 as runtime dtype ids
    assert C.tensor_capable_prims() == [0, 1, 3, 5, 6, 2, 4]
    d = C.runtime_dir()
    assert os.path.isabs(d) and os.path.exists(os.path.join(d, "chelis_device_owner.h"))


def test_host_program_lowers_only_its_count_helpers():
    """lib.rs:229-300: the Count-bearing helper becomes a HIP translation
    unit under its own name; the softmax helper keeps its C-host disposition."""
    g = DB.Dag("count")
    b = g.load("b", [64, 300], "bool")
    g.roots = [g.node({"Count": {"axes": [1]}}, [b], [64], "i64")]
    helpers = [("row_counts", g.json()), ("probs", DB.softmax_program(4, 8, "f32").json())]
    out = C.codegen_hip_host_program(helpers)
    assert [n for n, _ in out] == ["row_counts"]
    r = out[0][1]
    assert "extern \"C\" void row_counts_device(" in r.c_source and r.input_labels == ["b"]


# ---------------------------------------------------------------- comparison, cast, integer, gather regions
def region_kinds(prog):
    return [line.split()[1] for line in prog.describe().splitlines()]


def test_select_cast_integer_and_gather_regions_plan_one_launch_per_node():
    """Compare / Logical / Where / Cast / integer arithmetic / Gather stay
    their own node (fuse.rs:76-96 fuses none of them, and excludes integer
    sub, abs, max_elem and min_elem), one launch each, as the reference HIP
    lane emits them (kernels.rs:1270-1346, 1382, 769-866, 2557-2597)."""
    def load(name):
        return C.DagProgram(open(os.path.join(DAGS, name + ".json")).read())
    assert region_kinds(load("select_rows_f32_4096x1024")) == ["compare", "compare", "logical", "logical", "where",
                                                               "compare"]
    assert region_kinds(load("casts_f64_65536")) == ["chain", "cast", "cast", "cast"]
    assert region_kinds(load("integer_ops_i64_65536")) == ["integer"] * 5
    p = load("gathers_50000x64_4096x10")
    assert region_kinds(p) == ["gather", "gather"]
    assert [o[1] for o in p.outputs] == [(4096, 64), (4096, 1)]


def test_new_ops_read_and_write_back_verbatim():
    """Logical, Gather and Mod payloads survive the reader and the fuse pass's
    writer unchanged (the serde forms of dag.rs:553-559, 1349-1356)."""
    g = DB.Dag("ops")
    a = g.load("a", [4, 6], "f32")
    i = g.load("i", [3], "i64")
    x = g.load("x", [3], "i64")
    c = g.compare("lt", a, a)
    g.roots = [g.logical("not", c), g.gather(a, i, 1), g.binary("Mod", x, x), g.logical("or", c, c)]
    out = json.loads(C.dag_fuse(g.json()))
    assert [n["op"] for n in out["nodes"]][3:] == [{"Compare": "lt"}, {"Logical": "not"},
                                                    {"Gather": {"axis": 1, "batch_rank": 0}}, "Mod",
                                                    {"Logical": "or"}]


def test_an_integer_fused_chain_is_refused_as_both_reference_lanes_refuse_it():
    """fuse.rs joins integer add and mul into a FusedElem; the C lane rejects
    integer chains (crates/chelis-backend-c/src/emit.rs:6933-6945) and the HIP
    lane has no integer chain kernel, so the planner refuses them too. The
    same ops apart (a fan-out between them) plan as integer launches."""
    g = DB.Dag("int_chain")
    a, b, c = (g.load(n, [16], "i64") for n in "abc")
    g.roots = [g.add(g.mul(a, b), c)]
    with pytest.raises(C.ChelisError, match="integer fused elementwise chain"):
        C.DagProgram(g.json())
    g = DB.Dag("int_apart")
    a, b = (g.load(n, [16], "i64") for n in "ab")
    m = g.mul(a, b)
    g.roots = [m, g.add(m, b)]
    assert region_kinds(C.DagProgram(g.json())) == ["integer", "integer"]


def test_generated_entries_read_the_failure_record_only_when_a_launch_traps():
    src = C.CodegenResult(open(os.path.join(DAGS, "integer_ops_i64_65536.json")).read(), "f").c_source
    assert "chelis_hip_take_numeric_failure" in src and "chelis_numeric_trap(chelis_failure.message)" in src
    src = C.CodegenResult(open(os.path.join(DAGS, "select_rows_f32_4096x1024.json")).read(), "f").c_source
    assert "chelis_hip_take_numeric_failure" not in src


def test_draw_keys_derive_while_planning_or_are_refused():
    """key_from_seed / split / fold_in of literals are derived while planning
    and take no launch (emit.rs:3594-3653); a run-time seed, or a derived key
    read as a value, is refused as the reference refuses it."""
    p = C.DagProgram(open(os.path.join(DAGS, "draws_f32_1024x512.json")).read())
    assert region_kinds(p) == ["uniform_like", "dropout"]
    g = DB.Dag("runtime_seed")
    s = g.load("s", [], "i64")
    x = g.load("x", [8], "f32")
    k = g.node("KeyFromSeed", [s], [], "key")
    g.roots = [g.uniform_like(x, 0.0, 1.0, k)]
    with pytest.raises(C.ChelisError, match="run-time seed"):
        C.DagProgram(g.json())
    g = DB.Dag("key_result")
    g.roots = [g.key_from_seed(5)]
    with pytest.raises(C.ChelisError, match="derived key as a result"):
        C.DagProgram(g.json())
    p = C.DagProgram(open(os.path.join(DAGS, "extrema_adjoints_f32_4096x1024.json")).read())
    assert region_kinds(p) == ["extrema_adjoint"] * 3


def test_cumsum_plans_as_a_scan_and_reads_back_verbatim():
    p = C.DagProgram(open(os.path.join(DAGS, "scans_f32_512x1024.json")).read())
    assert region_kinds(p) == ["cumsum"] * 3
    g = DB.Dag("scan")
    x = g.load("x", [3, 4], "i8")
    g.roots = [g.cumsum(x, 0, "Decreasing")]
    out = json.loads(C.dag_fuse(g.json()))
    assert out["nodes"][1]["op"] == {"Cumsum": {"axis": 0, "direction": "Decreasing"}}
    assert out["nodes"][1]["output_type"]["precision"] == "Int32"


def test_bitwise_pad_shrink_stride_plan_and_read_back_verbatim():
    p = C.DagProgram(open(os.path.join(DAGS, "bitwise_i32_65536.json")).read())
    assert region_kinds(p) == ["integer"] * 5
    p = C.DagProgram(open(os.path.join(DAGS, "movement_f32_512x1000.json")).read())
    assert region_kinds(p) == ["chain", "pad", "copy", "copy"]
    text = open(os.path.join(DAGS, "movement_f32_512x1000.json")).read()
    assert json.loads(C.dag_fuse(text))["nodes"][1]["op"] == {
        "Shrink": {"bounds": [[{"Lit": 10}, {"Lit": 490}], [{"Lit": 100}, {"Lit": 1000}]]}}


def test_movement_bounds_this_build_refuses():
    g = DB.Dag("bad")
    x = g.load("x", [8, 6], "f32")
    g.roots = [g.shrink(x, [(2, 9), (0, 6)])]  # past the operand
    with pytest.raises(C.ChelisError, match="Shrink bounds outside the operand on axis 0"):
        C.DagProgram(g.json())
    g = DB.Dag("bad")
    x = g.load("x", [8, 6], "f32")
    n = g.stride(x, [3, 2])
    g.nodes[n]["output_type"]["dims"][0] = {"Lit": 2}  # ceil(8 / 3) is 3
    g.roots = [n]
    with pytest.raises(C.ChelisError, match="bounds do not give the node's extent on axis 0"):
        C.DagProgram(g.json())
    g = DB.Dag("bad")
    x = g.load("x", [8, 6], "f32")
    k = g.const(2, [], "i64")
    n = g.node({"Shrink": {"bounds": [[{"Node": 1}, {"Lit": 8}], [{"Lit": 0}, {"Lit": 6}]]}}, [x, k], [6, 6], "f32")
    g.roots = [n]
    with pytest.raises(C.ChelisError, match="run-time bounds"):
        C.DagProgram(g.json())


def test_scatters_plan_one_launch_each():
    p = C.DagProgram(open(os.path.join(DAGS, "scatters_5000x64_4096.json")).read())
    assert region_kinds(p) == ["scatter"] * 3
    text = open(os.path.join(DAGS, "scatters_5000x64_4096.json")).read()
    nodes = json.loads(C.dag_fuse(text))["nodes"]
    assert [list(n["op"])[0] for n in nodes[6:]] == ["ScatterAdd", "Scatter", "ScatterElements"]


def test_literal_tensors_sit_in_the_constant_pool():
    text = open(os.path.join(DAGS, "literals_f32_256x1000.json")).read()
    p = C.DagProgram(text)
    assert region_kinds(p) == ["chain", "integer", "copy"]
    assert C.dag_fuse(text).count('"ConstTensor"') == 2
    g = DB.Dag("bad")
    g.roots = [g.const_tensor([1.0, 2.0, 3.0], [4], "f32")]  # three values for four elements
    with pytest.raises(C.ChelisError, match="ConstTensor data does not fill"):
        C.DagProgram(g.json())

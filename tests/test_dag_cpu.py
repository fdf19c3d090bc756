"""The DAG front end on the host (no GPU): the reference's wire form read
and written back byte for byte, fuse.rs's chain rules, the region plans of
the configuration programs, unsupported ops named, and the codegen surface
(its source compiles against the library's headers)."""
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


def test_plans_of_the_configuration_programs():
    assert kinds(plan("softmax_f32_16384x1024")) == ["softmax"]
    assert kinds(plan("gemm_f32_4096")) == ["matmul"]
    assert kinds(plan("linreg_step_8192x32")) == ["matmul", "chain", "matmul", "chain", "reduce", "chain"]
    t = plan("transformer_block_b8_s512_d1024")
    # the scores product, causal softmax and P.V fold into one attention region
    assert kinds(t) == ["layer_norm", "matmul", "matmul", "matmul", "attention", "matmul", "layer_norm", "matmul",
                        "matmul"]
    desc = t.describe().splitlines()
    assert "causal" in desc[4] and "permuted" in desc[4]
    assert "bias gelu" in desc[7] and "bias residual" in desc[8] and "-> output 0" in desc[8]
    # the slot plan reuses ranges: four slots, three of [4096, 1024] f32 and
    # one holding the [4096, 4096] FFN hidden layer; no score tensor
    n_const = sum(1 for n in json.load(open(os.path.join(DAGS, "transformer_block_b8_s512_d1024.json")))["nodes"]
                  if isinstance(n["op"], dict) and "Const" in n["op"])
    assert t.peak_device_bytes == 3 * 8 * 512 * 1024 * 4 + 8 * 512 * 4096 * 4 + 8 * n_const
    m = plan("mlp_train_step_1024x784x512x10")
    k = kinds(m)
    assert k.count("matmul") == 5 and k.count("softmax") == 1 and k.count("softmax_adjoint") == 1
    assert k.count("dropout") == 2 and k.count("relu") == 1 and k.count("relu_adjoint") == 1
    assert [o[0] for o in m.outputs] == ["out0", "out1", "out2", "out3", "out4"]
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
    assert r.input_labels == ["X", "w", "y"] and r.output_labels == ["out0", "out1"]
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

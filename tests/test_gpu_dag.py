"""The DAG front end on the GPU (include/chelis_dag.h): programs read from
lowered DAGs in the reference's wire form (tests/golden/dags/, written by
tests/golden/dag_builder.py) run through the planned regions and match the
C oracle to the same bar as the hand-wired programs, and the hand-wired
programs' bits where the launch sequence is the same."""
import json
import os
import sys

import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import dag_builder as DB  # noqa: E402

DAGS = os.path.join(HERE, "golden", "dags")


def setup_module(_m):
    O.build()


def fixture(name):
    with open(os.path.join(DAGS, name + ".json")) as fh:
        return fh.read()


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def normwise(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-300))


@pytest.mark.parametrize("name,dtype,rows,n", [("softmax_f32_16384x1024", np.float32, 16384, 1024),
                                               ("softmax_f64_4096x4096", np.float64, 4096, 4096)])
def test_softmax_config2_from_dag(name, dtype, rows, n):
    p = C.DagProgram(fixture(name))
    assert p.launches == 1
    x = (np.random.default_rng(10).standard_normal((rows, n)) * 2).astype(dtype)
    ref = O.softmax_rows(x)
    prev = C.set_exact(True)
    try:
        (y,) = p.run([C.to_device(x)])
    finally:
        C.set_exact(prev)
    assert bits_equal(y.numpy(), ref)
    # the default mode: binary32 unchanged, binary64 the faithful row
    (y,) = p.run([C.to_device(x)])
    if dtype == np.float32:
        assert bits_equal(y.numpy(), ref)
    else:
        assert normwise(y.numpy(), ref) <= 1e-13


@pytest.mark.parametrize("m,n,k,dtype", [(256, 192, 320, np.float64), (512, 512, 256, np.float32),
                                         (1000, 64, 777, np.float64), (300, 1, 513, np.float64)])
def test_matmul_from_dag_is_the_dispatch(m, n, k, dtype):
    """A lowered matmul runs as one launch of the matmul dispatch: the same
    bits as chelis_hip_matmul, and within the GEMM tolerance of the
    canonical-tree oracle (bit-exact on the tree-kernel shapes)."""
    prec = "f32" if dtype == np.float32 else "f64"
    p = C.DagProgram(DB.matmul_program(m, n, k, prec).json())
    rng = np.random.default_rng(m + n + k)
    a, b = rng.uniform(-1, 1, (m, k)).astype(dtype), rng.uniform(-1, 1, (k, n)).astype(dtype)
    da, db = C.to_device(a), C.to_device(b)
    (c,) = p.run([da, db])
    direct = C.matmul(da, db)
    assert bits_equal(c.numpy(), direct.numpy())
    ref = O.matmul(a, b)
    tol = 1e-5 if dtype == np.float32 else 1e-10
    assert normwise(c.numpy(), ref) <= tol


def linreg_inputs(n=8192, d=32):
    X = np.random.default_rng(1).standard_normal((n, d))
    w = np.random.default_rng(2).standard_normal(d)
    y = X @ w + np.random.default_rng(3).normal(0, 0.01, n)
    return X, w, y


def reversed_roots(name):
    """The fixture with its roots reversed: planned region by region (not as
    the recognized whole program), the outputs in reverse order."""
    d = json.loads(fixture(name))
    d["roots"] = d["roots"][::-1]
    return json.dumps(d)


@pytest.mark.parametrize("whole", [True, False])
def test_linreg_config1_from_dag_bit_exact(whole):
    """As the recognized program (the fused two-launch step) and region by
    region: the same bits as the oracle either way."""
    p = C.DagProgram(fixture("linreg_step_8192x32") if whole else reversed_roots("linreg_step_8192x32"))
    assert p.launches == (1 if whole else 6)
    X, w, y = linreg_inputs()
    outs = p.run([C.to_device(a) for a in (X, w, y)])
    grad, loss = outs if whole else outs[::-1]
    g_ref, l_ref = O.linreg_step(X, w, y)
    assert bits_equal(grad.numpy(), g_ref) and bits_equal(loss.numpy(), np.float64(l_ref))


def transformer_inputs(B, S, D, F):
    x = np.random.default_rng(30).standard_normal((B, S, D)).astype(np.float32)
    p = {}
    seeds = iter(range(31, 37))
    for name, shape in (("wq", (D, D)), ("wk", (D, D)), ("wv", (D, D)), ("wo", (D, D)), ("w1", (D, F)),
                        ("w2", (F, D))):
        p[name] = (np.random.default_rng(next(seeds)).standard_normal(shape) * 0.02).astype(np.float32)
    for name, n in (("bq", D), ("bk", D), ("bv", D), ("bo", D), ("b1", F), ("b2", D), ("ln1_b", D), ("ln2_b", D)):
        p[name] = np.random.default_rng(n + len(name)).standard_normal(n).astype(np.float32) * 0.1
    p["ln1_g"] = 1 + np.random.default_rng(5).standard_normal(D).astype(np.float32) * 0.1
    p["ln2_g"] = 1 + np.random.default_rng(6).standard_normal(D).astype(np.float32) * 0.1
    return x, p


@pytest.mark.parametrize("dims", [(2, 128, 256, 1024), (8, 512, 1024, 4096)])
def test_transformer_config4_from_dag(dims):
    """Seven regions (Q, K and V as one batched product; the attention
    scores, causal softmax and P.V fused into one): the launches of the
    hand-wired chelis_prog_transformer_block, so its bits, and within 1e-5
    of the oracle normwise and elementwise (relative, with an absolute
    floor of 1e-5: the block's output carries the unit-scale residual)."""
    B, S, D, F = dims
    text = fixture("transformer_block_b8_s512_d1024") if dims == (8, 512, 1024, 4096) else \
        DB.transformer_program(B, S, D, F).json()
    prog = C.DagProgram(text)
    assert prog.launches == 7
    x, p = transformer_inputs(B, S, D, F)
    ins = [C.to_device(x)] + [C.to_device(p[k]) for k in DB.TRANSFORMER_PARAMS]
    (y,) = prog.run(ins)
    hand = C.empty(x.shape, np.float32)
    C.program("transformer_block", ins, [hand])
    assert bits_equal(y.numpy(), hand.numpy())
    ref = O.transformer_block(x, p, D // 64)
    assert normwise(y.numpy(), ref) <= 1e-5
    err = np.abs(y.numpy().astype(np.float64) - ref) / (np.abs(ref) + 1.0)
    assert err.max() <= 1e-5, float(err.max())


def mlp_inputs(B=1024, I=784, H=512, O_=10):
    x = np.random.default_rng(40).uniform(0, 1, (B, I)).astype(np.float32)
    labels = np.random.default_rng(41).integers(0, O_, B)
    onehot = np.eye(O_, dtype=np.float32)[labels]
    w1 = (np.random.default_rng(42).standard_normal((I, H)) * np.sqrt(2 / I)).astype(np.float32)
    w2 = (np.random.default_rng(43).standard_normal((H, O_)) * np.sqrt(2 / H)).astype(np.float32)
    return x, onehot, w1, np.zeros(H, np.float32), w2, np.zeros(O_, np.float32)


@pytest.mark.parametrize("whole", [True, False])
@pytest.mark.parametrize("exact", [True, False])
def test_mlp_config5_from_dag(exact, whole):
    """As the recognized program (the five-launch step) and region by region."""
    prog = C.DagProgram(fixture("mlp_train_step_1024x784x512x10") if whole else
                        reversed_roots("mlp_train_step_1024x784x512x10"))
    assert (prog.launches == 1) == whole
    args = mlp_inputs()
    ref = O.mlp_train_step(*args, 44, np.float32(0.1), np.float32(0.01))
    prev = C.set_exact_matmul(exact)
    try:
        outs = prog.run([C.to_device(a) for a in args] + [C.key_tensor(44)])
        got = [o.numpy() for o in (outs if whole else outs[::-1])]
    finally:
        C.set_exact_matmul(prev)
    if exact:
        for g, r, name in zip(got, ref, ("loss", "w1", "b1", "w2", "b2")):
            assert bits_equal(np.asarray(g, np.float32), np.asarray(r, np.float32)), (name, normwise(g, r))
        return
    for g, r, name in zip(got[1:], ref[1:], ("w1", "b1", "w2", "b2")):
        assert normwise(g, r) <= 1e-5, name


def test_strided_inputs_and_reshape_views():
    """Inputs may be any strided views: a transposed operand through the
    matmul, and a reshape that is not one run of memory is refused."""
    m, k, n = 64, 48, 40
    p = C.DagProgram(DB.matmul_program(m, n, k, "f64").json())
    rng = np.random.default_rng(3)
    at = rng.standard_normal((k, m))
    b = rng.standard_normal((k, n))
    dat = C.to_device(at)
    a_view = dat.view((m, k), (1, m))
    (c,) = p.run([a_view, C.to_device(b)])
    assert normwise(c.numpy(), at.T @ b) <= 1e-12
    g = DB.Dag("flat")
    x = g.load("x", [4, 6], "f64")
    g.roots = [g.add(g.reshape(x, [24]), g.const(1.0, [24], "f64"))]
    prog = C.DagProgram(g.json())
    xs = rng.standard_normal((6, 4))
    with pytest.raises(C.ChelisError, match="not one run of memory"):
        prog.run([C.to_device(xs).view((4, 6), (1, 4))])
    (y,) = prog.run([C.to_device(xs.T.copy())])
    assert np.array_equal(y.numpy(), xs.T.reshape(24) + 1.0)


def test_generic_regions_every_op_kind():
    """A DAG of the generic kinds: a chain over broadcast and constant
    operands, a chain inlined into a sum, max / min / prod / argmax
    reductions, relu and its adjoint, dropout and its replay, a count."""
    g = DB.Dag("generic")
    x = g.load("x", [64, 300], "f32")
    y = g.load("y", [300], "f32")
    key = g.load("key", [], "key")
    ye = g.expand_to_match(y, [64, 300])
    t = g.unary("Sqrt", g.unary("Abs", g.sub(x, ye)))
    s = g.sum(g.mul(t, t), 1)
    mx = g.max_reduce(x, 1)
    mn = g.node({"MinReduce": {"axis": 0}}, [x], [300], "f32")
    am = g.node({"Argmax": {"axis": 1}}, [x], [64], "i64")
    r = g.relu(x)
    ra = g.relu_adjoint(x, g.neg(x))
    rate = g.const(0.25, [], "f32")
    d = g.dropout(x, rate, key)
    dr = g.dropout(x, rate, key, replay=True)
    g.roots = [t, s, mx, mn, am, r, ra, d, dr]
    prog = C.DagProgram(g.json())
    rng = np.random.default_rng(8)
    xv = rng.standard_normal((64, 300)).astype(np.float32)
    yv = rng.standard_normal(300).astype(np.float32)
    outs = [o.numpy() for o in prog.run([C.to_device(xv), C.to_device(yv), C.key_tensor(77)])]
    tv = np.sqrt(np.abs(xv - yv)).astype(np.float32)
    assert bits_equal(outs[0], tv)
    assert bits_equal(outs[1], O.sum_axis((tv * tv).astype(np.float32), 1))
    assert bits_equal(outs[2], O.max_axis(xv, 1))
    assert bits_equal(outs[3], -O.max_axis(-xv, 0))
    assert np.array_equal(outs[4], np.argmax(xv, 1))
    assert bits_equal(outs[5], O.relu(xv))
    assert bits_equal(outs[6], O.relu_adjoint(xv, -xv))
    assert bits_equal(outs[7], O.dropout(77, xv, np.float32(0.25)))
    assert bits_equal(outs[8], O.dropout_replay(77, xv, np.float32(0.25)))


def test_count_region_reports_through_the_trap_channel():
    """A Count region runs without waiting; a byte other than 0 / 1 is read
    from the trap channel once after the run and raised there; the channel
    is clear for the next run."""
    g = DB.Dag("count")
    b = g.load("b", [64, 300], "bool")
    c = g.node({"Count": {"axes": [1]}}, [b], [64], "i64")
    g.roots = [c]
    prog = C.DagProgram(g.json())
    bits = (np.random.default_rng(3).random((64, 300)) < 0.3).astype(np.uint8)
    (y,) = prog.run([C.to_device(bits)])
    assert np.array_equal(y.numpy(), bits.sum(1))
    bad = bits.copy()
    bad[5, 7] = 2
    with pytest.raises(C.ChelisError, match="domain in count at bool"):
        prog.run([C.to_device(bad)])
    (y,) = prog.run([C.to_device(bits)])
    assert np.array_equal(y.numpy(), bits.sum(1))


def test_mlp_program_region_refuses_strided_outputs():
    """The recognized MLP step writes dense results, as every chain region
    does: an output given as a strided view is refused before any launch,
    and dense outputs then run."""
    prog = C.DagProgram(fixture("mlp_train_step_1024x784x512x10"))
    args = mlp_inputs()
    ins = [C.to_device(a) for a in args] + [C.key_tensor(44)]
    outs = prog.empty_outputs()
    big = C.empty((512, 784), np.float32)
    outs[1] = big.view((784, 512), (1, 784))
    with pytest.raises(C.ChelisError, match="writes dense results"):
        prog.run(ins, outs)
    dense = [o.numpy() for o in prog.run(ins)]
    assert all(np.isfinite(d).all() for d in dense)

"""The generated entries on the GPU: chelis_codegen_hip's C++ for each
configuration DAG (tests/golden/dags/) compiled with its own compile and
link flags, loaded, and called through {f}_device (device owners in and
out) and {f} (host tensors in and out) - the functions `chelis build
--target hip` hands a caller (crates/chelis-backend-hip/src/emit.rs:667-808,
838-964) - checked against the C oracle to the same bar as the program
tests; and one compiled program with run-time extents run at several sizes."""
import os
import sys
import tempfile

import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import dag_builder as DB  # noqa: E402
from test_gpu_dag import linreg_inputs, mlp_inputs, transformer_inputs  # noqa: E402

DAGS = os.path.join(HERE, "golden", "dags")
_TMP = tempfile.TemporaryDirectory()
_BUILT = {}


def setup_module(_m):
    O.build()


def fixture(name):
    with open(os.path.join(DAGS, name + ".json")) as fh:
        return fh.read()


def generated(name, text=None):
    """The compiled generated program of a fixture (built once per run)."""
    if name not in _BUILT:
        _BUILT[name] = C.GeneratedProgram(text or fixture(name), "gen_" + name, _TMP.name)
    return _BUILT[name]


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def normwise(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-300))


@pytest.mark.parametrize("entry", ["device", "host"])
def test_linreg_config1_generated_entries_bit_exact(entry):
    g = generated("linreg_step_8192x32")
    assert g.result.input_labels == ["X", "w", "y"] and g.result.output_labels == ["root0", "root1"]
    X, w, y = linreg_inputs()
    if entry == "device":
        grad, loss = [t.numpy() for t in g.device([C.to_device(a) for a in (X, w, y)])]
    else:
        grad, loss = g.host([X, w, y])
    g_ref, l_ref = O.linreg_step(X, w, y)
    assert bits_equal(grad, g_ref) and bits_equal(np.asarray(loss, np.float64), np.float64(l_ref))


@pytest.mark.parametrize("entry", ["device", "host"])
@pytest.mark.parametrize("name,dtype,rows,n", [("softmax_f32_16384x1024", np.float32, 16384, 1024),
                                               ("softmax_f64_4096x4096", np.float64, 4096, 4096)])
def test_softmax_config2_generated_entries(entry, name, dtype, rows, n):
    g = generated(name)
    x = (np.random.default_rng(10).standard_normal((rows, n)) * 2).astype(dtype)
    ref = O.softmax_rows(x)
    prev = C.set_exact(True)
    try:
        y = g.device([C.to_device(x)])[0].numpy() if entry == "device" else g.host([x])[0]
    finally:
        C.set_exact(prev)
    assert y.shape == (rows, n) and bits_equal(y, ref)
    y = g.device([C.to_device(x)])[0].numpy() if entry == "device" else g.host([x])[0]
    if dtype == np.float32:
        assert bits_equal(y, ref)
    else:
        assert normwise(y, ref) <= 1e-13


@pytest.mark.parametrize("name,m,n,k,dtype", [("gemm_f32_4096", 4096, 4096, 4096, np.float32),
                                              ("gemm_f64_4096", 4096, 4096, 4096, np.float64),
                                              ("skinny_f64_8192x64x4096", 8192, 64, 4096, np.float64),
                                              ("gemv_f64_8192", 8192, 1, 8192, np.float64)])
def test_matmul_config3_generated_device_entry(name, m, n, k, dtype):
    """The dispatch's bits (the same launch as chelis_hip_matmul), and the
    GEMM tolerance against the canonical-tree oracle on sampled rows."""
    g = generated(name)
    rng = np.random.default_rng(20 + m + n + k)
    a, b = rng.uniform(-1, 1, (m, k)).astype(dtype), rng.uniform(-1, 1, (k, n)).astype(dtype)
    da, db = C.to_device(a), C.to_device(b)
    (c,) = g.device([da, db])
    c = c.numpy()
    assert c.shape == (m, n)
    assert bits_equal(c, C.matmul(da, db).numpy())
    rows = np.concatenate([[0, m - 1], np.random.default_rng(0).choice(m, 30, replace=False)])
    ref = O.matmul(np.ascontiguousarray(a[rows]), b)
    tol = 1e-5 if dtype == np.float32 else 1e-10
    assert normwise(c[rows], ref) <= tol
    assert np.all(np.abs(c[rows] - ref) <= tol * np.abs(b).max() * np.abs(a[rows]).sum(1, keepdims=True))


@pytest.mark.parametrize("entry", ["device", "host"])
def test_transformer_config4_generated_entries(entry):
    """Within 1e-5 of the oracle normwise, and elementwise within 1e-5
    relative with an absolute floor of 1e-5 (the block's output has unit
    scale: it adds the residual stream x ~ N(0, 1))."""
    g = generated("transformer_block_b8_s512_d1024")
    x, p = transformer_inputs(8, 512, 1024, 4096)
    arrays = [x] + [p[k] for k in DB.TRANSFORMER_PARAMS]
    if entry == "device":
        (y,) = [t.numpy() for t in g.device([C.to_device(a) for a in arrays])]
    else:
        (y,) = g.host(arrays)
    ref = O.transformer_block(x, p, 16)
    assert normwise(y, ref) <= 1e-5
    err = np.abs(y.astype(np.float64) - ref) / (np.abs(ref) + 1.0)
    assert err.max() <= 1e-5, float(err.max())


@pytest.mark.parametrize("entry", ["device", "host"])
def test_mlp_config5_generated_entries_bit_exact(entry):
    g = generated("mlp_train_step_1024x784x512x10")
    args = mlp_inputs()
    ref = O.mlp_train_step(*args, 44, np.float32(0.1), np.float32(0.01))
    prev = C.set_exact_matmul(True)
    try:
        if entry == "device":
            got = [t.numpy() for t in g.device([C.to_device(a) for a in args] + [C.key_tensor(44)])]
        else:
            got = g.host(list(args) + [("key", 44)])
    finally:
        C.set_exact_matmul(prev)
    for gv, r, name in zip(got, ref, ("loss", "w1", "b1", "w2", "b2")):
        assert bits_equal(np.asarray(gv, np.float32), np.asarray(r, np.float32)), (name, normwise(gv, r))


# ---------------------------------------------------------------- run-time extents
@pytest.mark.parametrize("name,shapes", [("softmax_f32_rows_x1024", [(300, 1024), (16384, 1024), (1, 1024)]),
                                         ("softmax_f32_rows_x_cols", [(77, 333), (4096, 1024), (5, 4096)])])
def test_one_program_with_run_time_extents_runs_at_several_sizes(name, shapes):
    """One compiled program (and one generated entry) binds its run-time
    extents from each call's input and matches the oracle bit for bit."""
    p = C.DagProgram(fixture(name))
    g = generated(name)
    assert g.result.symbolic_dims == p.symbolic_dims != []
    for shape in shapes:
        x = (np.random.default_rng(shape[0]).standard_normal(shape) * 2).astype(np.float32)
        ref = O.softmax_rows(x)
        (y,) = p.run([C.to_device(x)])
        assert y.shape == shape and bits_equal(y.numpy(), ref), shape
        (yd,) = g.device([C.to_device(x)])
        assert bits_equal(yd.numpy(), ref), shape
        (yh,) = g.host([x])
        assert bits_equal(yh, ref), shape


def test_a_run_time_sized_workspace_slot_at_two_sizes():
    """A softmax whose result is read by a chain: the intermediate takes a
    workspace range sized 4096 * rows at each call."""
    gb = DB.Dag("sym")
    x = gb.load("x", ["rows", 1024], "f32")
    sm = gb.softmax(x, 1)
    gb.roots = [gb.add(sm, sm)]
    p = C.DagProgram(gb.json())
    assert p.peak_device_bytes == -1
    for rows in (3, 5000):
        xv = np.random.default_rng(rows).standard_normal((rows, 1024)).astype(np.float32)
        s = O.softmax_rows(xv)
        (y,) = p.run([C.to_device(xv)])
        assert bits_equal(y.numpy(), (s + s).astype(np.float32))


@pytest.mark.parametrize("name", ["linreg_step_8192x32", "mlp_train_step_1024x784x512x10", "gemm_f64_4096"])
def test_prepared_dag_runs_the_same_bits(name):
    """prepare_dag_for_codegen's BlasMatmul nodes plan to the same launches
    as the lowered matmuls they replace: identical results."""
    text = fixture(name)
    a, b = C.DagProgram(text), C.DagProgram(C.prepare_dag_for_codegen(text))
    if name.startswith("linreg"):
        ins = [C.to_device(v) for v in linreg_inputs()]
    elif name.startswith("mlp"):
        ins = [C.to_device(v) for v in mlp_inputs()] + [C.key_tensor(44)]
    else:
        rng = np.random.default_rng(5)
        ins = [C.to_device(rng.uniform(-1, 1, (4096, 4096))) for _ in range(2)]
    for x, y in zip(a.run(ins), b.run(ins)):
        assert bits_equal(x.numpy(), y.numpy())

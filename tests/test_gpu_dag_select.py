"""The comparison / logical / where, checked-cast, checked-integer and gather
region kinds through the DAG path (chelis_dag_run) and the generated entries
({f}_device and {f}), against the C oracle bit for bit. A failing element
reaches the caller as the reference's trap line: a ChelisError from the
DAG run, and from a generated entry the line on stderr with exit status 1
([04-NUM-10]'s boundary; crates/chelis-runtime/include/chelis_runtime.h:
73-82), for the earliest failing launch at its lowest failing element."""
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import dag_builder as DB  # noqa: E402

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
DAGS = os.path.join(HERE, "golden", "dags")
_TMP = tempfile.TemporaryDirectory()
_BUILT = {}


def setup_module(_m):
    O.build()


def fixture(name):
    with open(os.path.join(DAGS, name + ".json")) as fh:
        return fh.read()


def generated(name):
    if name not in _BUILT:
        _BUILT[name] = C.GeneratedProgram(fixture(name), "gen_" + name.split("_")[0], _TMP.name)
    return _BUILT[name]


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8).tobytes()


def run_dag(name, arrays):
    prog = C.DagProgram(fixture(name))
    return [t.numpy() for t in prog.run([C.to_device(a) for a in arrays])]


def run_all(name, arrays):
    """The outputs through the DAG run, the device entry and the host entry."""
    g = generated(name)
    return {"dag": run_dag(name, arrays),
            "device": [t.numpy() for t in g.device([C.to_device(a) for a in arrays])],
            "host": g.host(arrays)}


# ---------------------------------------------------------------- select rows
def select_inputs(R=4096, N=1024):
    rng = np.random.default_rng(60)
    x = rng.standard_normal((R, N)).astype(np.float32)
    y = rng.standard_normal((R, N)).astype(np.float32)
    t = (rng.standard_normal(N) * 0.5).astype(np.float32)
    x[0, :8] = [np.nan, -0.0, 0.0, np.inf, -np.inf, 1.0, t[6], 2.0]
    y[0, :8] = [1.0, 0.0, -0.0, np.nan, -1.0, -0.0, np.nan, -np.inf]
    return x, y, t


def select_oracle(x, y, t):
    R, N = x.shape
    above = O.compare("gt", "f32", x, np.broadcast_to(t, (R, N)))
    negative = O.compare("lt", "f32", y, np.zeros((R, N), np.float32))
    keep = O.logical("and", above, O.logical("not", negative))
    w = O.where(keep, x, y)
    return [w, keep, O.compare("eq", "f32", w, x)]


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_select_rows_bit_exact(path):
    x, y, t = select_inputs()
    got = run_all("select_rows_f32_4096x1024", [x, y, t])[path]
    for g, w in zip(got, select_oracle(x, y, t)):
        assert bits(g) == bits(w)


# ---------------------------------------------------------------- casts
def cast_inputs(n=65536, bad=None):
    rng = np.random.default_rng(61)
    x = rng.standard_normal(n) * 10.0 ** rng.integers(-5, 9, n)
    x[:12] = [0.5, 1.5, 2.5, -0.5, -2.5, 1e-320, -0.0, 1.5e9 + 0.5, 1.0 + 2.0 ** -8 + 2.0 ** -40,
              65519.99, 2147483647.4, -2147483648.49]
    if bad is not None:
        x[bad] = np.nan
    return x


def round_half_even(x):
    """RiscOp::Round is the C lane's rint: halves to even
    (crates/chelis-backend-c/src/emit.rs:2434)."""
    return np.rint(x)


def cast_oracle(x):
    return [O.cast("f64", "i32", round_half_even(x)), O.cast("f64", "f32", x), O.cast("f64", "bf16", x)]


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_casts_bit_exact(path):
    x = cast_inputs()
    got = run_all("casts_f64_65536", [x])[path]
    want = cast_oracle(x)
    for g, (w, first, _) in zip(got, want):
        assert first == -1
        assert bits(g) == bits(w)


def test_round_helper_matches_the_device_round():
    """The test's round against the library's own round step, so the cast
    check above is not resting on an assumption."""
    x = cast_inputs()
    out = C.empty(x.shape, np.float64)
    C.fused_elementwise(C.fused_chain([("round", 0)]), [C.to_device(x)], out)
    assert bits(out.numpy()) == bits(round_half_even(x))


# ---------------------------------------------------------------- integer ops
def integer_inputs(n=65536, zero_at=None):
    rng = np.random.default_rng(62)
    a = rng.integers(-(2 ** 62), 2 ** 62, n, dtype=np.int64)
    b = rng.integers(-1000, 1000, n, dtype=np.int64)
    b[b == 0] = 7
    a[:6] = [7, 7, -7, -7, -(2 ** 62), 5]  # the fifth: a - floor_div(a, -1) is exactly i64's minimum
    b[:6] = [2, -2, 2, -2, -1, 3]
    if zero_at is not None:
        b[zero_at] = 0
    return a, b


def integer_oracle(a, b):
    steps = [("floor_div", "q", "a", "b"), ("mod", "r", "a", "b"), ("max_elem", "m", "q", "r"),
             ("sub", "d", "a", "m"), ("trunc_div", "t", "a", "b")]
    env = {"a": a, "b": b}
    for op, dst, x, y in steps:
        env[dst], first, _ = O.int_binary(op, "i64", env[x], env[y])
        assert first == -1, (op, first)
    return [env["q"], env["r"], env["d"], env["t"]]


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_integer_ops_bit_exact(path):
    a, b = integer_inputs()
    got = run_all("integer_ops_i64_65536", [a, b])[path]
    for g, w in zip(got, integer_oracle(a, b)):
        assert np.array_equal(g, w)


def test_integer_trap_through_the_dag_run():
    a, b = integer_inputs(zero_at=[40000, 777])
    with pytest.raises(C.ChelisError, match="^numeric trap: division by zero in floor_div at i64$"):
        run_dag("integer_ops_i64_65536", [a, b])
    # the record was read and cleared: the next run is clean
    a, b = integer_inputs()
    run_dag("integer_ops_i64_65536", [a, b])


# ---------------------------------------------------------------- gathers
def gather_inputs(bad=False):
    rng = np.random.default_rng(63)
    table = rng.standard_normal((50000, 64)).astype(np.float32)
    ids = rng.integers(0, 50000, 4096).astype(np.int64)
    logits = rng.standard_normal((4096, 10)).astype(np.float32)
    labels = rng.integers(0, 10, (4096, 1)).astype(np.int64)
    if bad:
        labels[100, 0] = 10
    return table, ids, logits, labels


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_gathers_bit_exact(path):
    table, ids, logits, labels = gather_inputs()
    got = run_all("gathers_50000x64_4096x10", [table, ids, logits, labels])[path]
    assert bits(got[0]) == bits(O.gather(table, ids, 0)[0])
    assert bits(got[1]) == bits(O.gather(logits, labels, 1, batch_rank=1)[0])
    assert np.array_equal(got[0], table[ids]) and np.array_equal(got[1][:, 0], logits[np.arange(4096), labels[:, 0]])


# ---------------------------------------------------------------- generated entries trap
CHILD = r"""
import sys, numpy as np
sys.path.insert(0, sys.argv[1])
import ctypes, chelis_amd as C
lib = ctypes.CDLL(sys.argv[2])
case = sys.argv[3]
if case == "integer":
    n = 65536
    a = np.arange(n, dtype=np.int64) - 3
    b = np.ones(n, np.int64)
    b[[50000, 9]] = 0
    C.host_entry(sys.argv[4], [a, b], 4, library=lib)
elif case == "cast":
    x = np.zeros(65536)
    x[[3000, 70]] = [np.inf, 3e9]
    C.host_entry(sys.argv[4], [x], 3, library=lib)
elif case == "shift":
    n = 65536
    a = np.arange(n, dtype=np.int32)
    c = np.ones(n, np.int32)
    c[[40000, 12]] = [-1, -4]
    C.host_entry(sys.argv[4], [a, a, c], 5, library=lib)
elif case == "scatter":
    table = np.zeros((5000, 64), np.float32)
    ids = np.zeros(4096, np.int64)
    ids[[3000, 40]] = [5000, -3]
    C.host_entry(sys.argv[4], [table, ids, np.zeros((4096, 64), np.float32), np.zeros((512, 100), np.float32),
                               np.zeros((512, 30), np.int32), np.zeros((512, 30), np.float32)], 3, library=lib)
elif case == "gather":
    table = np.zeros((50000, 64), np.float32)
    ids = np.zeros(4096, np.int64)
    ids[17] = -1
    logits = np.zeros((4096, 10), np.float32)
    labels = np.zeros((4096, 1), np.int64)
    outs = C.device_entry(sys.argv[4], [C.to_device(v) for v in (table, ids, logits, labels)], 2, library=lib)
print("returned", flush=True)
"""


@pytest.mark.parametrize("name,case,text", [
    ("integer_ops_i64_65536", "integer", "numeric trap: division by zero in floor_div at i64"),
    ("casts_f64_65536", "cast", "numeric trap: overflow in cast at i32"),
    ("gathers_50000x64_4096x10", "gather", "numeric trap: domain in gather at i64"),
    ("bitwise_i32_65536", "shift", "shift amount must be non-negative, got -4"),
    ("scatters_5000x64_4096", "scatter", "numeric trap: domain in scatter at i64"),
])
def test_generated_entries_exit_with_the_trap_line(name, case, text):
    g = generated(name)
    r = subprocess.run([sys.executable, "-c", CHILD, os.path.dirname(HERE), g.path, case, g.name],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 1, (r.returncode, r.stdout[-1000:], r.stderr[-2000:])
    assert text in r.stderr and "returned" not in r.stdout


# ---------------------------------------------------------------- keyed draws, extrema cotangent
@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_draws_with_plan_derived_keys_bit_exact(path):
    """key_from_seed(1234), split, fold_in(7) derived while planning
    ([05-OP-69..72]), then uniform_like(-1, 2) and dropout(0.1) on the
    device: the oracle's draws from the same derived keys, bit for bit."""
    x = np.random.default_rng(64).standard_normal((1024, 512)).astype(np.float32)
    got = run_all("draws_f32_1024x512", [x])[path]
    left, right = O.split(1234)
    u = O.uniform_like(O.fold_in(left, 7), -1.0, 2.0, x.size, np.float32).reshape(x.shape)
    assert bits(got[0]) == bits(u)
    assert bits(got[1]) == bits(O.dropout(right, x, np.float32(0.1)))


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_extrema_adjoints_bit_exact(path):
    rng = np.random.default_rng(65)
    a = rng.standard_normal((4096, 1024)).astype(np.float32)
    b = a.copy()
    b[::2] = rng.standard_normal((2048, 1024)).astype(np.float32)  # half the rows tie exactly
    a[0, :4] = [np.nan, 0.0, -0.0, np.inf]
    b[0, :4] = [1.0, -0.0, 0.0, np.nan]
    g = rng.standard_normal((4096, 1024)).astype(np.float32)
    got = run_all("extrema_adjoints_f32_4096x1024", [a, b, g])[path]
    want = [O.extrema_adjoint("max", "left", "f32", a, b, g), O.extrema_adjoint("max", "right", "f32", a, b, g),
            O.extrema_adjoint("min", "left", "f32", a, b, g)]
    for x, y in zip(got, want):
        assert bits(x) == bits(y)


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_scans_bit_exact(path):
    rng = np.random.default_rng(66)
    x = rng.standard_normal((512, 1024)).astype(np.float32)
    c = rng.integers(-10 ** 12, 10 ** 12, 512).astype(np.int64)
    got = run_all("scans_f32_512x1024", [x, c])[path]
    want = [O.cumsum("f32", x, 1)[0], O.cumsum("f32", x, 0, reverse=True)[0], O.cumsum("i64", c, 0)[0]]
    for g, w in zip(got, want):
        assert bits(g) == bits(w)


def test_scan_overflow_traps_through_the_dag_run():
    x = np.zeros((512, 1024), np.float32)
    c = np.zeros(512, np.int64)
    c[[7, 8]] = np.iinfo(np.int64).max
    with pytest.raises(C.ChelisError, match="^numeric trap: overflow in cumsum at i64$"):
        run_dag("scans_f32_512x1024", [x, c])


# ---------------------------------------------------------------- bitwise, movement
def bitwise_inputs(n=65536):
    rng = np.random.default_rng(67)
    a = rng.integers(-(2 ** 31), 2 ** 31, n, dtype=np.int64).astype(np.int32)
    b = rng.integers(-(2 ** 31), 2 ** 31, n, dtype=np.int64).astype(np.int32)
    c = rng.integers(0, 40, n).astype(np.int32)
    c[:4] = [0, 31, 32, 1000]
    a[:4] = [-1, -(2 ** 31), 5, -7]
    return a, b, c


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_bitwise_bit_exact(path):
    a, b, c = bitwise_inputs()
    got = run_all("bitwise_i32_65536", [a, b, c])[path]
    want = [O.int_binary(op, "i32", a, y)[0] for op, y in
            (("bitand", b), ("bitxor", b), ("bitor", b), ("shl", c), ("shr", c))]
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_negative_shift_count_through_the_dag_run():
    a, b, c = bitwise_inputs()
    c[[900, 300]] = [-5, -2]
    with pytest.raises(C.ChelisError, match="^shift amount must be non-negative, got -2$"):
        run_dag("bitwise_i32_65536", [a, b, c])


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_movement_views_and_pad_bit_exact(path):
    """Shrink and stride as views (an offset, scaled strides) read by a
    chain, a pad of the chain's result, and a stride and a shrink written
    out by copies."""
    x = np.random.default_rng(68).standard_normal((512, 1000)).astype(np.float32)
    got = run_all("movement_f32_512x1000", [x])[path]
    s = O.slice_(x, [10, 100], [1, 1], [480, 900])
    t = O.slice_(s, [0, 0], [3, 2], [160, 450])
    y = t + np.float32(1.0)
    want = [O.pad(y, [2, 0], [1, 5], np.float32(-1.5)), O.slice_(x, [0, 0], [2, 5], [256, 200]),
            O.slice_(x, [500, 0], [1, 1], [12, 1000])]
    for g, w in zip(got, want):
        assert g.shape == w.shape and bits(g) == bits(w)


# ---------------------------------------------------------------- scatters
def scatter_inputs(bad_col=False):
    rng = np.random.default_rng(69)
    table = rng.standard_normal((5000, 64)).astype(np.float32)
    ids = rng.integers(0, 700, 4096).astype(np.int64)
    grads = rng.standard_normal((4096, 64)).astype(np.float32)
    data = rng.standard_normal((512, 100)).astype(np.float32)
    cols = rng.integers(0, 100, (512, 30)).astype(np.int32)
    if bad_col:
        cols[9, 4] = 100
    vals = rng.standard_normal((512, 30)).astype(np.float32)
    return [table, ids, grads, data, cols, vals]


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_scatters_bit_exact(path):
    table, ids, grads, data, cols, vals = ins = scatter_inputs()
    got = run_all("scatters_5000x64_4096", ins)[path]
    want = [O.scatter("f32", table, ids, grads, 0, add=True)[0], O.scatter("f32", table, ids, grads, 0)[0],
            O.scatter_elements("f32", data, cols, vals, 1)[0]]
    for g, w in zip(got, want):
        assert bits(g) == bits(w)


def test_scatter_elements_trap_through_the_dag_run():
    with pytest.raises(C.ChelisError, match="^numeric trap: domain in scatter_elements at i64$"):
        run_dag("scatters_5000x64_4096", scatter_inputs(bad_col=True))


@pytest.mark.parametrize("path", ["dag", "device", "host"])
def test_literal_tensors_bit_exact(path):
    """ConstTensor literals in the constant pool: a row read through an
    Expand by a chain, an i32 tensor as a result and as an operand; a Drop
    moves nothing."""
    rng = np.random.default_rng(70)
    x = rng.standard_normal((256, 1000)).astype(np.float32)
    y = rng.integers(-1000, 1000, (3, 4)).astype(np.int32)
    got = run_all("literals_f32_256x1000", [x, y])[path]
    row = np.float32(np.arange(1000)) * np.float32(0.37) - np.float32(100.5)
    grid = (np.arange(12).reshape(3, 4) * 7 - 40).astype(np.int32)
    assert bits(got[0]) == bits(x + row[None, :])
    assert np.array_equal(got[1], grid)
    assert np.array_equal(got[2], O.int_binary("bitxor", "i32", y, grid)[0])


def test_shrink_over_a_run_time_axis_at_two_sizes():
    """A shrink whose row bound runs to the end of a run-time extent
    ((0, ToEnd), spec/05 section 2.4.1) and whose column bounds are
    literal, read by a chain: one plan runs at two row counts."""
    g = DB.Dag("shrink_rt")
    x = g.load("x", ["rows", 1000], "f32")
    n = g.node({"Shrink": {"bounds": [[{"Lit": 0}, "ToEnd"], [{"Lit": 100}, {"Lit": 900}]]}}, [x], ["rows", 800],
               "f32")
    g.roots = [g.binary("Mul", n, g.scalar_like(2.0, n))]
    prog = C.DagProgram(g.json())
    for rows in (64, 300):
        xs = np.random.default_rng(rows).standard_normal((rows, 1000)).astype(np.float32)
        got = prog.run([C.to_device(xs)])[0].numpy()
        want = O.slice_(xs, [0, 100], [1, 1], [rows, 800]) * np.float32(2.0)
        assert got.shape == (rows, 800) and bits(got) == bits(want)

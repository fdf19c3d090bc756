"""GPU parity of comparison, logical, where, checked casts, checked integer
arithmetic and gather (chelis_hip_compare / logical / where / cast /
integer_elementwise / gather) against the C oracle: every result bit for
bit, every failure at the oracle's lowest failing index with its kind and
[04-NUM-9]'s trap line; broadcast and strided operands; the deferred record
keeps the earliest failing launch."""
import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f64": np.float64, "bf16": np.uint16, "f16": np.float16, "i8": np.int8, "i16": np.int16,
      "i32": np.int32, "i64": np.int64, "bool": np.uint8}
DTS = list(NP)


def setup_module(_m):
    O.build()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def sample(dt, n, rng):
    """n values of dtype dt with the specials its casts and comparisons
    turn on (NaN payloads, signed zeros, infinities, range ends, ties)."""
    if dt in ("f32", "f64"):
        sp = [0.0, -0.0, 1.0, -1.0, 0.5, 2.5, -2.5, np.inf, -np.inf, np.nan, 127.0, 128.0, -129.0, 32767.0,
              2147483647.0, 2147483648.0, -2147483648.0, 9.3e18, -9.223372036854775808e18, 65504.0, 65520.0, 1e-40,
              3.4e38, 1.0 + 2.0 ** -8 + 2.0 ** -30, 255.0, 1e300]
        x = np.concatenate([np.array(sp), rng.standard_normal(n) * 10.0 ** rng.integers(-3, 12, n)])
        x = x.astype(NP[dt])
        if dt == "f32":
            x.view(np.uint32)[-3:] = [0x7FC00001, 0xFF800001, 0x80000001]
        return x
    if dt == "bf16":
        return np.concatenate([np.array([0, 0x8000, 0x3F80, 0x7F80, 0xFF80, 0x7FC1, 0x4300, 0x4700, 0xC700, 1],
                                        np.uint16), rng.integers(0, 65536, n).astype(np.uint16)])
    if dt == "f16":
        b = np.concatenate([np.array([0, 0x8000, 0x3C00, 0x7C00, 0xFC00, 0x7E01, 0x5800, 0x7BFF, 1], np.uint16),
                            rng.integers(0, 65536, n).astype(np.uint16)])
        return b.view(np.float16)
    if dt == "bool":
        return rng.integers(0, 2, n + 4).astype(np.uint8)
    info = np.iinfo(NP[dt])
    edge = np.array([info.min, info.min + 1, -1, 0, 1, 2, 127, 128, -129, 255, info.max], np.int64)
    edge = edge[(edge >= info.min) & (edge <= info.max)].astype(NP[dt])
    small = rng.integers(-300, 300, n // 2)
    small = small[(small >= info.min) & (small <= info.max)].astype(NP[dt])
    return np.concatenate([edge, small, rng.integers(info.min, info.max, n // 2, dtype=NP[dt], endpoint=True)])


def oracle_carrier(dt, x):
    return x.view(np.uint16) if dt == "f16" else x


# ---------------------------------------------------------------- compare / logical / where
@pytest.mark.parametrize("dt", [d for d in DTS if d != "bool"])
def test_compare_every_kind(dt):
    rng = np.random.default_rng(DTS.index(dt))
    v = sample(dt, 120, rng)
    a = np.repeat(v, 37)[: 4001]
    b = np.tile(v, 37)[: 4001]
    rng.shuffle(b)
    da, db = C.to_device(a), C.to_device(b)
    for kind in C.COMPARE_KINDS:
        got = C.compare(kind, da, db).numpy()
        want = O.compare(kind, dt, oracle_carrier(dt, a), oracle_carrier(dt, b))
        assert np.array_equal(got, want), (dt, kind)


def test_compare_bool_and_broadcast():
    rng = np.random.default_rng(1)
    a = rng.integers(0, 2, (33, 65)).astype(np.uint8)
    b = rng.integers(0, 2, (1, 65)).astype(np.uint8)
    for kind in ("eq", "neq"):
        assert np.array_equal(C.compare(kind, C.to_device(a), C.to_device(b)).numpy(), O.compare(kind, "bool", a, b))
    x = rng.standard_normal((4, 1, 300)).astype(np.float32)
    y = rng.standard_normal((4, 7, 1)).astype(np.float32)
    got = C.compare("gte", C.to_device(x), C.to_device(y)).numpy()
    assert got.shape == (4, 7, 300)
    assert np.array_equal(got, O.compare("gte", "f32", x, y))
    with pytest.raises(C.ChelisError):
        C.compare("lt", C.to_device(a), C.to_device(b))


def test_compare_of_a_transposed_view():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((300, 200)).astype(np.float64)
    d = C.to_device(x)
    t = d.view((200, 300), (1, 200))
    y = rng.standard_normal((200, 300))
    got = C.compare("lt", t, C.to_device(y)).numpy()
    assert np.array_equal(got, O.compare("lt", "f64", np.ascontiguousarray(x.T), y))


def test_logical():
    rng = np.random.default_rng(3)
    a = rng.choice(np.array([0, 1, 2, 255], np.uint8), (5, 1000))
    b = rng.choice(np.array([0, 1, 2, 255], np.uint8), (5, 1000))
    da, db = C.to_device(a), C.to_device(b)
    for kind in ("and", "or"):
        assert np.array_equal(C.logical(kind, da, db).numpy(), O.logical(kind, a, b))
    assert np.array_equal(C.logical("not", da).numpy(), O.logical("not", a))


@pytest.mark.parametrize("dt", ["f32", "f64", "bf16", "i8", "i64", "bool"])
def test_where_selects_stored_bits(dt):
    rng = np.random.default_rng(4 + DTS.index(dt))
    a = sample(dt, 3000, rng)
    b = sample(dt, 3000, rng)[: len(a)]
    a = a[: len(b)]
    rng.shuffle(b)
    c = rng.integers(0, 3, len(a)).astype(np.uint8)
    got = C.where(C.to_device(c), C.to_device(a), C.to_device(b)).numpy()
    assert bits(got).tobytes() == bits(O.where(c, a, b)).tobytes()
    # broadcast branches: a row and a scalar
    c2 = rng.integers(0, 2, (64, 129)).astype(np.uint8)
    a2 = a[:129].reshape(1, 129)
    b2 = b[:1].reshape(1, 1)
    got = C.where(C.to_device(c2), C.to_device(a2), C.to_device(b2)).numpy()
    assert bits(got).tobytes() == bits(O.where(c2, a2, b2)).tobytes()


# ---------------------------------------------------------------- casts
@pytest.mark.parametrize("src", DTS)
def test_cast_to_every_dtype(src):
    rng = np.random.default_rng(10 + DTS.index(src))
    x = sample(src, 3000, rng)
    dx = C.to_device(x)
    for dst in DTS:
        want, first, kind = O.cast(src, dst, oracle_carrier(src, x))
        out, failure = C.cast(dx, NP[dst])
        got = out.numpy()
        assert bits(got).tobytes() == bits(want).tobytes(), (src, dst)
        if first < 0:
            assert failure is None, (src, dst, failure)
        else:
            assert failure == (first, kind, O.trap_text(kind, "cast", dst)), (src, dst, failure)


def test_cast_of_a_broadcast_view_and_the_lowest_offender():
    x = np.array([1.0, 2.0, 3.0, 1e20, 4.0, 0.5, 1e20, np.nan], np.float64)
    big = np.tile(x, 5000)
    out, failure = C.cast(C.to_device(big), np.int32)
    assert failure == (3, 1, "numeric trap: overflow in cast at i32")
    big[2] = np.nan
    _, failure = C.cast(C.to_device(big), np.int32)
    assert failure == (2, 2, "numeric trap: domain in cast at i32")
    row = C.to_device(np.array([[1.5, -2.0, 3.0]], np.float32))
    v = row.view((4, 3), (0, 1))
    out, failure = C.cast(v, np.float64)
    assert failure is None and np.array_equal(out.numpy(), np.tile([[1.5, -2.0, 3.0]], (4, 1)))


# ---------------------------------------------------------------- integer arithmetic
@pytest.mark.parametrize("dt", ["i8", "i16", "i32", "i64"])
def test_integer_binary_every_op(dt):
    rng = np.random.default_rng(20 + DTS.index(dt))
    v = sample(dt, 200, rng)
    a = np.repeat(v, len(v))
    b = np.tile(v, len(v))
    da, db = C.to_device(a), C.to_device(b)
    for op in O.INT_BINARY:
        want, first, kind = O.int_binary(op, dt, a, b)
        out, failure = C.integer_op(op, da, db)
        assert np.array_equal(out.numpy(), want), (dt, op)
        if first < 0:
            assert failure is None
        elif op in ("shl", "shr"):
            text = f"shift amount must be non-negative, got {int(b[first])}"
            assert failure == (first, kind, text), (dt, op, failure)
        else:
            assert failure == (first, kind, O.trap_text(kind, op, dt)), (dt, op, failure)


def test_shift_counts_broadcast_and_the_deferred_count_line():
    """A broadcast count row; through the deferred record the message
    still names the count at the earliest failing launch's lowest element."""
    x = np.arange(-40, 40, dtype=np.int16).reshape(8, 10)
    c = np.array([[0, 1, 3, 15, 16, 17, 100, 2, 5, 9]], np.int16)
    want, first, _ = O.int_binary("shr", "i16", x, np.broadcast_to(c, x.shape))
    out, failure = C.integer_op("shr", C.to_device(x), C.to_device(c))
    assert failure is None and np.array_equal(out.numpy(), want)
    bad = c.copy()
    bad[0, [6, 3]] = [-7, -2]
    C.take_numeric_failure()
    C.integer_op("add", C.to_device(x), C.to_device(x), deferred=True)
    C.integer_op("shl", C.to_device(x), C.to_device(bad), deferred=True)
    C.integer_op("shr", C.to_device(x), C.to_device(np.full((1, 10), -9, np.int16)), deferred=True)
    assert C.take_numeric_failure() == (3, 2, "shift amount must be non-negative, got -2")
    assert C.take_numeric_failure() is None


@pytest.mark.parametrize("dt", ["i8", "i32", "i64"])
def test_integer_unary_and_broadcast(dt):
    rng = np.random.default_rng(30)
    x = sample(dt, 500, rng)
    for op in ("neg", "abs"):
        want, first, kind = O.int_unary(op, dt, x)
        out, failure = C.integer_op(op, C.to_device(x))
        assert np.array_equal(out.numpy(), want)
        assert failure == (first, kind, O.trap_text(kind, op, dt))
    safe = np.clip(x, -11, 11).astype(NP[dt])
    m = safe[:60].reshape(6, 10)
    r = safe[60:70].reshape(1, 10)
    out, failure = C.integer_op("mul", C.to_device(m), C.to_device(r))
    assert failure is None and np.array_equal(out.numpy(), O.int_binary("mul", dt, m, r)[0])


def test_integer_known_answers_and_trap_lines():
    a = C.to_device(np.array([7, 7, -7, -7], np.int64))
    b = C.to_device(np.array([2, -2, 2, -2], np.int64))
    assert C.integer_op("floor_div", a, b)[0].numpy().tolist() == [3, -4, -4, 3]
    assert C.integer_op("trunc_div", a, b)[0].numpy().tolist() == [3, -3, -3, 3]
    assert C.integer_op("mod", a, b)[0].numpy().tolist() == [1, 1, -1, -1]
    z = C.to_device(np.array([1, 0, 1, 1], np.int64))
    assert C.integer_op("floor_div", a, z)[1] == (1, 3, "numeric trap: division by zero in floor_div at i64")
    i8a = C.to_device(np.array([100, 127], np.int8))
    i8b = C.to_device(np.array([50, 1], np.int8))
    assert C.integer_op("add", i8a, i8b)[1] == (0, 1, "numeric trap: overflow in add at i8")


# ---------------------------------------------------------------- gather
@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("vdt", [np.float32, np.float64, np.uint16, np.int8])
def test_gather_matches_the_oracle(vdt, itype):
    rng = np.random.default_rng(40)
    values = (rng.standard_normal((6, 50, 9)) * 100).astype(vdt)
    for axis in range(3):
        idx = rng.integers(0, values.shape[axis], (7, 3)).astype(itype)
        want, first, _ = O.gather(values, idx, axis)
        out, failure = C.gather(C.to_device(values), C.to_device(idx), axis)
        assert first == -1 and failure is None
        assert bits(out.numpy()).tobytes() == bits(want).tobytes()


def test_gather_batched_strided_and_failing():
    rng = np.random.default_rng(41)
    values = rng.standard_normal((4, 30, 5)).astype(np.float32)
    idx = rng.integers(0, 30, (4, 11)).astype(np.int64)
    want, _, _ = O.gather(values, idx, 1, batch_rank=1)
    out, failure = C.gather(C.to_device(values), C.to_device(idx), 1, batch_rank=1)
    assert failure is None and np.array_equal(out.numpy(), want)
    # values as a transposed view
    base = C.to_device(np.ascontiguousarray(values.transpose(2, 1, 0)))  # [5, 30, 4]
    view = base.view((4, 30, 5), (1, 4, 120))
    out, failure = C.gather(view, C.to_device(idx), 1, batch_rank=1)
    assert failure is None and np.array_equal(out.numpy(), want)
    bad = idx.copy()
    bad[2, 7] = 30
    bad[3, 0] = -1
    want, first, kind = O.gather(values, bad, 1, batch_rank=1)
    out, failure = C.gather(C.to_device(values), C.to_device(bad), 1, batch_rank=1)
    assert failure == (first, kind, "numeric trap: domain in gather at i64")
    assert np.array_equal(out.numpy(), want)
    with pytest.raises(C.ChelisError, match="domain in gather"):
        C.gather(C.to_device(values), C.to_device(idx[:3]), 1, batch_rank=1)


# ---------------------------------------------------------------- the deferred record
def test_deferred_record_keeps_the_earliest_failing_launch():
    assert C.take_numeric_failure() is None
    ok = C.to_device(np.arange(10, dtype=np.int32))
    C.integer_op("add", ok, ok, deferred=True)
    bad_late = C.to_device(np.array([0.0, 0.0, 0.0, 0.0, 0.0, np.nan], np.float64))
    bad_early = C.to_device(np.array([1, 2, 3, 0], np.int64))
    C.integer_op("trunc_div", bad_early, bad_early, deferred=True)  # division by zero at 3
    C.cast(bad_late, np.int64, deferred=True)  # domain at 5, a later launch
    assert C.take_numeric_failure() == (3, 3, "numeric trap: division by zero in trunc_div at i64")
    assert C.take_numeric_failure() is None
    C.cast(bad_late, np.int64, deferred=True)
    assert C.take_numeric_failure() == (5, 2, "numeric trap: domain in cast at i64")


@pytest.mark.parametrize("dt", ["f32", "f64", "bf16", "f16"])
def test_extrema_adjoint_every_kind_and_operand(dt):
    rng = np.random.default_rng(50 + DTS.index(dt))
    v = sample(dt, 60, rng)
    a = np.repeat(v, len(v))
    b = np.tile(v, len(v))
    g = sample(dt, len(a), rng)[: len(a)]
    da, db, dg = C.to_device(a), C.to_device(b), C.to_device(g)
    for kind in (0, 1):
        for operand in (0, 1):
            k, side = ("max", "min")[kind], ("left", "right")[operand]
            out = C.extrema_adjoint(k, side, da, db, dg)
            want = O.extrema_adjoint(k, side, dt, oracle_carrier(dt, a), oracle_carrier(dt, b), oracle_carrier(dt, g))
            assert bits(out.numpy()).tobytes() == bits(want).tobytes(), (dt, kind, operand)


# ---------------------------------------------------------------- ordered scan
@pytest.mark.parametrize("dt", ["f32", "f64", "bf16", "f16", "i8", "i16", "i32", "i64"])
@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_every_dtype_axis_and_direction(dt, reverse):
    rng = np.random.default_rng(70 + DTS.index(dt))
    if dt in ("f32", "f64"):
        x = (rng.standard_normal((6, 333, 70)) * 10.0 ** rng.integers(-3, 4, (6, 333, 70))).astype(NP[dt])
        x[0, 5, 3] = np.nan
    elif dt in ("bf16", "f16"):
        x = O.narrow_encode(dt, rng.standard_normal((6, 333, 70)).astype(np.float32))
        x = x.view(np.float16) if dt == "f16" else x
    else:
        x = rng.integers(-100, 100, (6, 333, 70)).astype(NP[dt])
    dx = C.to_device(x)
    for axis in range(3):
        want, first, _ = O.cumsum(dt, oracle_carrier(dt, x), axis, reverse)
        out, failure = C.cumsum(dx, axis, reverse)
        assert first == -1 and failure is None
        assert bits(out.numpy()).tobytes() == bits(want).tobytes(), (dt, axis, reverse)


def test_cumsum_overflow_in_the_lanes_order_and_a_strided_view():
    big = np.iinfo(np.int64).max
    x = np.zeros((4, 10, 3), np.int64)
    x[2, 0, 1], x[2, 1, 1] = big, 1       # line (o=2, j=1) overflows at step 1
    x[3, 0, 0], x[3, 4, 0] = big, 1       # a later line
    want, first, kind = O.cumsum("i64", x, 1)
    out, failure = C.cumsum(C.to_device(x), 1)
    assert failure == (first, kind, "numeric trap: overflow in cumsum at i64") and first == (2 * 3 + 1) * 10 + 1
    assert np.array_equal(out.numpy(), want)
    rng = np.random.default_rng(71)
    base = rng.standard_normal((64, 48)).astype(np.float32)
    d = C.to_device(base)
    v = d.view((48, 64), (1, 48))  # the transpose
    out, failure = C.cumsum(v, 1)
    assert failure is None and bits(out.numpy()).tobytes() == bits(O.cumsum("f32", np.ascontiguousarray(base.T), 1)[0]).tobytes()


# ---------------------------------------------------------------- pad
@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.uint16, np.int8, np.int32, np.int64])
def test_pad_matches_the_oracle(dtype):
    rng = np.random.default_rng(72)
    x = (rng.standard_normal((33, 1, 70)) * 40).astype(dtype)
    fill = dtype(5) if dtype != np.float32 else np.float32(-0.0)
    for lo, hi in (([0, 0, 0], [0, 0, 0]), ([2, 3, 1], [1, 0, 9]), ([0, 5, 64], [7, 2, 0])):
        out = C.pad(C.to_device(x), lo, hi, fill)
        assert bits(out.numpy()).tobytes() == bits(O.pad(x, lo, hi, fill)).tobytes(), (lo, hi)


def test_pad_of_a_transposed_view_into_a_strided_output():
    rng = np.random.default_rng(73)
    base = rng.standard_normal((40, 24)).astype(np.float64)
    v = C.to_device(base).view((24, 40), (1, 24))
    holder = C.empty((30, 2, 46), np.float64)
    out = holder.view((30, 46), (2 * 46, 1))  # every other [30, 46] plane row
    C.pad(v, [4, 1], [2, 5], 2.5, out=out)
    want = O.pad(np.ascontiguousarray(base.T), [4, 1], [2, 5], 2.5)
    got = holder.numpy()[:, 0, :]
    assert got.tobytes() == want.tobytes()


# ---------------------------------------------------------------- scatters
def _values(dt, shape, rng):
    """sample()'s values repeated to fill `shape`."""
    n = int(np.prod(shape))
    return np.resize(sample(dt, n, rng), n).reshape(shape)


def _scatter_case(dt, rng, shape, axis, ishape, batch_rank=0, itype=np.int64):
    target = _values(dt, shape, rng)
    if dt in ("i8", "i16", "i32", "i64"):
        target = np.clip(target, -20, 20).astype(NP[dt])
    idx = rng.integers(0, shape[axis], ishape).astype(itype)
    ushape = O.gather_shape(shape, ishape, axis, batch_rank)
    upd = _values(dt, ushape, rng)
    if dt in ("i8", "i16", "i32", "i64"):
        upd = np.clip(upd, -5, 5).astype(NP[dt])
    return target, idx, upd


@pytest.mark.parametrize("dt", ["f32", "f64", "bf16", "f16", "i8", "i16", "i32", "i64"])
@pytest.mark.parametrize("add", [False, True])
def test_scatter_matches_the_oracle(dt, add):
    rng = np.random.default_rng(80 + DTS.index(dt))
    for shape, axis, ishape, br, itype in (((50, 16), 0, (300,), 0, np.int64), ((6, 40, 5), 1, (7, 9), 0, np.int32),
                                           ((8, 30), 1, (8, 50), 1, np.int64), ((9,), 0, (400,), 0, np.int32)):
        target, idx, upd = _scatter_case(dt, rng, shape, axis, ishape, br, itype)
        want, first, _ = O.scatter(dt, oracle_carrier(dt, target), idx, oracle_carrier(dt, upd), axis, br, add=add)
        out, failure = C.scatter(C.to_device(target), C.to_device(idx), C.to_device(upd), axis, br, add=add)
        assert first == -1 and failure is None
        assert bits(out.numpy()).tobytes() == bits(want).tobytes(), (dt, add, shape, axis)


def test_scatter_add_long_runs_and_strided_updates():
    """Runs of thousands of updates on a few cells, and the updates as a
    transposed view: still the canonical tree in ascending position."""
    rng = np.random.default_rng(88)
    target = rng.standard_normal((4, 33)).astype(np.float32)
    idx = rng.integers(0, 4, 20000)
    base = (rng.standard_normal((33, 20000)) * 10.0 ** rng.integers(-4, 5, (33, 20000))).astype(np.float32)
    upd = C.to_device(base).view((20000, 33), (1, 20000))
    want, _, _ = O.scatter("f32", target, idx, np.ascontiguousarray(base.T), 0, add=True)
    out, failure = C.scatter(C.to_device(target), C.to_device(idx), upd, 0, add=True)
    assert failure is None and out.numpy().tobytes() == want.tobytes()


def test_scatter_embedding_gradient_shape():
    """The gather adjoint of the gathers fixture: 4096 ids into a
    [50000, 64] table."""
    rng = np.random.default_rng(89)
    table = np.zeros((50000, 64), np.float32)
    ids = rng.integers(0, 500, 4096)  # many repeats
    g = rng.standard_normal((4096, 64)).astype(np.float32)
    want, _, _ = O.scatter("f32", table, ids, g, 0, add=True)
    out, failure = C.scatter(C.to_device(table), C.to_device(ids), C.to_device(g), 0, add=True)
    assert failure is None and out.numpy().tobytes() == want.tobytes()


def test_scatter_failures_and_their_lines():
    t = C.to_device(np.zeros((10, 3), np.float32))
    idx = np.arange(70) % 10
    idx[[44, 5]] = [-1, 10]
    u = C.to_device(np.ones((70, 3), np.float32))
    _, f = C.scatter(t, C.to_device(idx), u, 0, add=True)
    assert f == (5 * 3, 2, "numeric trap: domain in scatter at i64")
    _, f = C.scatter(t, C.to_device(idx), u, 0)
    assert f == (5 * 3, 2, "numeric trap: domain in scatter_replace at i64")
    # an i16 tree that leaves the width at destination 3 (and later at 7)
    ti = np.zeros(10, np.int16)
    ii = np.array([3, 3, 7, 7, 1])
    ui = np.array([30000, 30000, 30000, 30000, 5], np.int16)
    want, first, kind = O.scatter("i16", ti, ii, ui, 0, add=True)
    _, f = C.scatter(C.to_device(ti), C.to_device(ii), C.to_device(ui), 0, add=True)
    assert f == (first, kind, "numeric trap: overflow in scatter at i16") and first == 5 + 3
    with pytest.raises(C.ChelisError, match="numeric trap: domain in scatter at i64"):
        C.scatter(t, C.to_device(np.zeros(4, np.int64)), C.to_device(np.ones((5, 3), np.float32)), 0, add=True)
    C.take_numeric_failure()
    C.scatter(t, C.to_device(idx), u, 0, add=True, deferred=True)
    assert C.take_numeric_failure() == (15, 2, "numeric trap: domain in scatter at i64")


@pytest.mark.parametrize("dt", ["f32", "i64", "bf16"])
def test_scatter_elements_matches_the_oracle(dt):
    rng = np.random.default_rng(90)
    data = _values(dt, (6, 7, 5), rng)
    for axis in range(3):
        ishape = (4, 3, 5) if axis != 2 else (6, 7, 9)
        idx = rng.integers(0, data.shape[axis], ishape)
        upd = _values(dt, ishape, rng)
        want, first, _ = O.scatter_elements(dt, oracle_carrier(dt, data), idx, oracle_carrier(dt, upd), axis)
        out, failure = C.scatter_elements(C.to_device(data), C.to_device(idx), C.to_device(upd), axis)
        assert first == -1 and failure is None
        assert bits(out.numpy()).tobytes() == bits(want).tobytes(), axis
    bad = np.zeros((6, 7, 5), np.int64)
    bad[1, 2, 3] = 7
    _, f = C.scatter_elements(C.to_device(data), C.to_device(bad), C.to_device(data), 2)
    assert f == ((1 * 7 + 2) * 5 + 3, 2, "numeric trap: domain in scatter_elements at i64")


# ---------------------------------------------------------------- empty and strided edges
def test_empty_operands_launch_nothing_and_keep_the_target():
    t = np.arange(12, dtype=np.float32).reshape(4, 3)
    out, f = C.scatter(C.to_device(t), C.to_device(np.zeros(0, np.int64)), C.to_device(np.zeros((0, 3), np.float32)),
                       0, add=True)
    assert f is None and np.array_equal(out.numpy(), t)
    out, f = C.scatter(C.to_device(t), C.to_device(np.zeros(0, np.int64)), C.to_device(np.zeros((0, 3), np.float32)),
                       0)
    assert f is None and np.array_equal(out.numpy(), t)
    out = C.pad(C.to_device(np.zeros((0, 5), np.float32)), [2, 1], [1, 0], 3.0)
    assert out.numpy().shape == (3, 6) and np.all(out.numpy() == 3.0)
    out, f = C.cumsum(C.to_device(np.zeros((3, 0, 2), np.int64)), 1)
    assert f is None and out.numpy().shape == (3, 0, 2)
    out, f = C.integer_op("shl", C.to_device(np.zeros(0, np.int32)), C.to_device(np.zeros(0, np.int32)))
    assert f is None and out.numpy().shape == (0,)


def test_scatter_from_strided_target_and_indices():
    rng = np.random.default_rng(91)
    base = rng.standard_normal((6, 40)).astype(np.float32)
    target = C.to_device(base).view((40, 6), (1, 40))  # the transpose
    idx_base = rng.integers(0, 40, (2, 30)).astype(np.int32)
    idx = C.to_device(idx_base).view((30,), (1,), 30)  # row 1 of the index array
    upd = rng.standard_normal((30, 6)).astype(np.float32)
    for add in (False, True):
        want, _, _ = O.scatter("f32", np.ascontiguousarray(base.T), idx_base[1], upd, 0, add=add)
        out, f = C.scatter(target, idx, C.to_device(upd), 0, add=add)
        assert f is None and out.numpy().tobytes() == want.tobytes()


def test_scatter_add_i8_tree_stays_in_range_where_a_left_fold_would_not():
    t = np.array([100, 0], np.int8)
    out, f = C.scatter(C.to_device(t), C.to_device(np.array([0, 0, 0])), C.to_device(np.array([27, 1, -1], np.int8)),
                       0, add=True)
    assert f is None and out.numpy().tolist() == [127, 0]


def test_cumsum_of_a_broadcast_view():
    row = np.array([1.5, -2.0, 0.25], np.float32)
    v = C.to_device(row).view((5, 3), (0, 1))
    out, f = C.cumsum(v, 0)
    assert f is None and out.numpy().tobytes() == O.cumsum("f32", np.broadcast_to(row, (5, 3)).copy(), 0)[0].tobytes()

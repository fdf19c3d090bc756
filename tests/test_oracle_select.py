"""Pins of the oracle's comparison, logical, where, checked cast, checked
integer arithmetic and gather functions. CPU only.

What pins what:
  compare: the spec's lowering table (spec/05-risc-primitives.md:1269-1281,
      [05-OP-36]) evaluated from exact rational order alone (fractions, NaN
      read from the bit pattern), so a signed-zero, NaN or operand-order
      mistake fails; bf16 decoded by a 16-bit shift through struct, f16 by
      numpy's binary16.
  logical: the truth tables of [05-OP-26..28] over bytes 0, 1, 2, 255.
  where: numpy's selection on the raw bit patterns (NaN payloads and -0).
  cast: float targets against an exact rational round-half-even restated
      from the IEEE format parameters (precision, exponent range,
      subnormal quantum, overflow threshold), and against numpy's own
      conversions where numpy rounds once (f64 -> f32, f64 -> f16); integer
      and bool targets against the boundary cases [04-NUM-14] and the C
      lane's runtime checks fix (chelis_runtime.h:209-273), including the
      lowest-index offender of [04-NUM-15].
  integer arithmetic: Python's unbounded integers with the width's range
      as the overflow test; the C lane's known answers for floor_div,
      trunc_div and mod (crates/chelis-backend-c/tests/exec_compile.rs:
      3338-3341, 3466-3560, 3389-3399) and its trap texts (:3691, 4902,
      4958, 12038).
  gather: numpy.take per batch, and the first out-of-range flat index.
"""
import math
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O


def setup_module(_m):
    O.build()


# ---------------------------------------------------------------- helpers
FORMATS = {  # precision p (significant bits), minimum normal exponent, maximum exponent
    "f64": (53, -1022, 1023), "f32": (24, -126, 127), "bf16": (8, -126, 127), "f16": (11, -14, 15)}


def rne(q: Fraction, fmt: str):
    """The value of format `fmt` nearest q, ties to the even significand;
    +-inf past the overflow threshold (max + half an ulp), exact zero kept
    with q's sign handled by the caller."""
    p, emin, emax = FORMATS[fmt]
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    quantum = Fraction(2) ** (max(e, emin) - p + 1)
    m = a / quantum
    lo = math.floor(m)
    r = m - lo
    k = lo + 1 if (r > Fraction(1, 2) or (r == Fraction(1, 2) and lo % 2 == 1)) else lo
    v = k * quantum
    big = (2 - Fraction(2) ** (1 - p)) * Fraction(2) ** emax
    if v > big:
        return sign * math.inf
    return sign * v


def bits16_value(bits: int, fmt: str):
    """Exact value of a 16-bit pattern (None for NaN)."""
    if fmt == "bf16":
        return struct.unpack("<f", struct.pack("<I", bits << 16))[0]
    return float(np.array([bits], np.uint16).view(np.float16)[0])


def value_bits16(v, fmt: str) -> int:
    """The 16-bit pattern of an exactly representable value (or +-inf, or
    +-0 with the sign of v)."""
    if fmt == "f16":
        return int(np.array([float(v)], np.float16).view(np.uint16)[0])
    b = struct.unpack("<I", struct.pack("<f", float(v)))[0]
    assert b & 0xFFFF == 0
    return b >> 16


def is_nan_bits(bits, fmt):
    if fmt == "bf16":
        return (bits & 0x7F80) == 0x7F80 and (bits & 0x7F) != 0
    return (bits & 0x7C00) == 0x7C00 and (bits & 0x3FF) != 0


# ---------------------------------------------------------------- compare
def _values(dt, rng):
    if dt in ("f32", "f64"):
        base = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 2.5, 1e-40, -1e-310, 3.0e38],
                        np.float64)
        x = np.concatenate([base, rng.standard_normal(30)]).astype(CAR[dt])
        return x
    if dt in ("bf16", "f16"):
        specials = [0x0000, 0x8000, 0x3F80 if dt == "bf16" else 0x3C00, 0x7F80 if dt == "bf16" else 0x7C00,
                    0xFF80 if dt == "bf16" else 0xFC00, 0x7FC0 if dt == "bf16" else 0x7E00, 0x0001, 0x8001]
        return np.concatenate([np.array(specials, np.uint16), rng.integers(0, 65536, 40).astype(np.uint16)])
    if dt == "bool":
        return np.array([0, 1, 0, 1, 1, 0], np.uint8)
    info = np.iinfo(CAR[dt])
    return np.concatenate([np.array([info.min, info.max, 0, -1, 1], CAR[dt]),
                           rng.integers(info.min, info.max, 30, dtype=CAR[dt], endpoint=True)])


CAR = {"f32": np.float32, "f64": np.float64, "i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64}


def _exact(dt, v):
    """(is NaN, exact value)."""
    if dt in ("bf16", "f16"):
        if is_nan_bits(int(v), dt):
            return True, None
        f = bits16_value(int(v), dt)
        return False, (f if math.isinf(f) else Fraction(f))
    if dt in ("f32", "f64"):
        if np.isnan(v):
            return True, None
        if np.isinf(v):
            return False, (math.inf if v > 0 else -math.inf)
        return False, Fraction(float(v))
    return False, Fraction(int(v))


def _cmplt(x, y):
    return x < y  # exact order of rationals / infinities


@pytest.mark.parametrize("dt", ["f32", "f64", "bf16", "f16", "i8", "i16", "i32", "i64"])
def test_compare_follows_the_lowering_table(dt):
    rng = np.random.default_rng(3)
    v = _values(dt, rng)
    a = np.repeat(v, len(v))
    b = np.tile(v, len(v))
    got = {k: O.compare(k, dt, a, b) for k in O.COMPARE_KINDS}
    for i in range(len(a)):
        na, x = _exact(dt, a[i])
        nb, y = _exact(dt, b[i])
        nan = na or nb
        lt = (not nan) and _cmplt(x, y)
        gt = (not nan) and _cmplt(y, x)
        want = {"cmp_lt": lt, "lt": lt, "eq": (not nan) and not (lt or gt), "neq": nan or lt or gt,
                "gt": gt, "gte": (not nan) and not lt, "lte": (not nan) and not gt}
        for k in want:
            assert got[k][i] == int(want[k]), (dt, k, a[i], b[i])


def test_bool_equality_on_stored_bytes():
    a = np.array([0, 1, 0, 1], np.uint8)
    b = np.array([0, 0, 1, 1], np.uint8)
    assert O.compare("eq", "bool", a, b).tolist() == [1, 0, 0, 1]
    assert O.compare("neq", "bool", a, b).tolist() == [0, 1, 1, 0]


def test_compare_broadcasts():
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = np.array([[1.0], [4.0]], np.float32)
    assert O.compare("lt", "f32", a, b).tolist() == [[1, 0, 0], [1, 0, 0]]


# ---------------------------------------------------------------- logical / where
def test_logical_truth_tables():
    bytes_ = np.array([0, 1, 2, 255], np.uint8)
    a = np.repeat(bytes_, 4)
    b = np.tile(bytes_, 4)
    assert O.logical("and", a, b).tolist() == [int(x != 0 and y != 0) for x, y in zip(a, b)]
    assert O.logical("or", a, b).tolist() == [int(x != 0 or y != 0) for x, y in zip(a, b)]
    assert O.logical("not", bytes_).tolist() == [1, 0, 0, 0]


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.uint16, np.int8, np.int64])
def test_where_keeps_the_selected_bits(dtype):
    rng = np.random.default_rng(4)
    n = 257
    if np.dtype(dtype).kind == "f":
        a = rng.standard_normal(n).astype(dtype)
        b = rng.standard_normal(n).astype(dtype)
        ub = np.uint32 if dtype == np.float32 else np.uint64
        a.view(ub)[:5] = np.array([0x7FC00001 if dtype == np.float32 else 0x7FF8000000000001, 0x80000000
                                   if dtype == np.float32 else 0x8000000000000000, 0, 1, 2], ub)
    else:
        a = rng.integers(0, 100, n).astype(dtype)
        b = rng.integers(0, 100, n).astype(dtype)
    c = rng.integers(0, 3, n).astype(np.uint8)
    got = O.where(c, a, b)
    want = np.where(c != 0, a, b)
    assert got.tobytes() == want.tobytes()


# ---------------------------------------------------------------- casts
def _float_sample(rng):
    xs = [0.0, -0.0, 1.0, -1.5, math.inf, -math.inf, 65504.0, 65520.0, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8,
          2.99e-8, 3.4e38, 3.4028235677973366e38, 3.4028235e38, 1e-39, 1e-45, 1.4e-45, 7e-46, 2.0 ** -149,
          2.0 ** -150, 2.0 ** -150 * 1.0000001, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -9, 1.0 + 2.0 ** -11,
          1.0 + 2.0 ** -11 + 2.0 ** -40, 1.0 + 2.0 ** -8 + 2.0 ** -40, 1e300, -1e-300]
    return np.concatenate([np.array(xs), rng.standard_normal(200) * 10.0 ** rng.integers(-40, 40, 200)])


def _expect_float_bits(q, fmt, negzero):
    v = rne(q, fmt) if q != 0 else 0
    if fmt == "f64":
        return struct.unpack("<Q", struct.pack("<d", -0.0 if negzero else float(v)))[0]
    if fmt == "f32":
        return struct.unpack("<I", struct.pack("<f", -0.0 if negzero else float(v)))[0]
    if v == 0 and negzero:
        return 0x8000
    if v == 0 and q != 0 and q < 0:
        return 0x8000
    return value_bits16(v, fmt)


@pytest.mark.parametrize("dst", ["f32", "bf16", "f16"])
def test_float_narrowing_rounds_once_to_nearest_even(dst):
    rng = np.random.default_rng(5)
    x = _float_sample(rng)
    y, first, _ = O.cast("f64", dst, x)
    assert first == -1
    ybits = y.view(np.uint32 if dst == "f32" else np.uint16)
    for i, v in enumerate(x):
        if math.isinf(v):
            q = None
        else:
            q = Fraction(float(v))
        if q is None:
            want = {"f32": 0x7F800000, "bf16": 0x7F80, "f16": 0x7C00}[dst] | (
                {"f32": 0x80000000, "bf16": 0x8000, "f16": 0x8000}[dst] if v < 0 else 0)
        else:
            want = _expect_float_bits(q, dst, math.copysign(1.0, v) < 0 and v == 0)
            if q < 0 and rne(q, dst) == 0:
                want = 0x80000000 if dst == "f32" else 0x8000
        assert int(ybits[i]) == want, (dst, v, hex(int(ybits[i])), hex(want))


@pytest.mark.filterwarnings("ignore:overflow encountered in cast")
def test_float_narrowing_matches_numpy_single_roundings():
    rng = np.random.default_rng(6)
    x = _float_sample(rng)
    y32, _, _ = O.cast("f64", "f32", x)
    assert y32.tobytes() == x.astype(np.float32).tobytes()
    y16, _, _ = O.cast("f64", "f16", x)
    assert y16.tobytes() == x.astype(np.float16).view(np.uint16).tobytes()
    x32 = x.astype(np.float32)
    z16, _, _ = O.cast("f32", "f16", x32)
    assert z16.tobytes() == x32.astype(np.float64).astype(np.float16).view(np.uint16).tobytes()


def test_nan_becomes_the_canonical_quiet_nan():
    x = np.array([0x7FF0000000000001, 0xFFF8000000000000], np.uint64).view(np.float64)
    for dst, want in (("f32", 0x7FC00000), ("bf16", 0x7FC0), ("f16", 0x7E00)):
        y, _, _ = O.cast("f64", dst, x)
        assert set(y.view(np.uint32 if dst == "f32" else np.uint16).tolist()) == {want}
    y, _, _ = O.cast("f32", "f64", np.array([0xFFC00001], np.uint32).view(np.float32))
    assert y.view(np.uint64)[0] == 0x7FF8000000000000
    same, _, _ = O.cast("f32", "f32", np.array([0xFFC00001], np.uint32).view(np.float32))
    assert same.view(np.uint32)[0] == 0xFFC00001  # an identity cast keeps the stored bits


@pytest.mark.parametrize("dst", ["f64", "f32", "bf16", "f16"])
def test_integer_to_float_rounds_once(dst):
    rng = np.random.default_rng(7)
    big = [2 ** 62 + 2 ** 54 + 1, 2 ** 62 + 2 ** 54, 2 ** 62 + 3 * 2 ** 54, -(2 ** 63), 2 ** 63 - 1, 2 ** 53 + 1,
           2 ** 24 + 1, 2 ** 24 + 3, 65519, 65520, 65505, 257, 258, 259, 0, -1]
    x = np.concatenate([np.array(big, np.int64), rng.integers(-(2 ** 63), 2 ** 63 - 1, 300, dtype=np.int64)])
    y, first, _ = O.cast("i64", dst, x)
    assert first == -1
    width = {"f64": np.uint64, "f32": np.uint32, "bf16": np.uint16, "f16": np.uint16}[dst]
    for i, v in enumerate(x.tolist()):
        q = rne(Fraction(v), dst) if v else 0
        if dst == "f64":
            want = struct.unpack("<Q", struct.pack("<d", float(q)))[0]
        elif dst == "f32":
            want = struct.unpack("<I", struct.pack("<f", float(q)))[0]
        else:
            want = value_bits16(q, dst) if not (isinstance(q, float) and math.isinf(q)) else (
                value_bits16(q, dst))
        assert int(y.view(width)[i]) == want, (dst, v)


CASES_TO_INT = [
    # (source, target, value, expected kind or value)
    ("f64", "i32", 2147483647.0, 2147483647), ("f64", "i32", 2147483648.0, "overflow"),
    ("f64", "i32", -2147483648.0, -2147483648), ("f64", "i32", -2147483649.0, "overflow"),
    ("f64", "i64", 9223372036854775808.0, "overflow"), ("f64", "i64", -9223372036854775808.0, -(2 ** 63)),
    ("f64", "i8", 127.0, 127), ("f64", "i8", 128.0, "overflow"), ("f64", "i8", -0.0, 0),
    ("f64", "i16", 0.5, "domain"), ("f64", "i16", math.inf, "domain"), ("f64", "i16", math.nan, "domain"),
    ("f64", "i64", 1e300, "overflow"), ("f64", "i64", -1e-300, "domain"),
    ("f32", "i32", 2147483648.0, "overflow"), ("f32", "i32", 2147483520.0, 2147483520),
    ("f32", "bool", 1.0, 1), ("f32", "bool", -0.0, 0), ("f32", "bool", 2.0, "domain"),
    ("f32", "bool", math.nan, "domain"), ("f64", "bool", 0.999, "domain"),
    ("i64", "i32", 2 ** 31, "overflow"), ("i64", "i32", -(2 ** 31), -(2 ** 31)), ("i32", "i8", -129, "overflow"),
    ("i16", "i64", -32768, -32768), ("i64", "bool", 1, 1), ("i64", "bool", 2, "domain"), ("i8", "bool", -1, "domain"),
    ("bool", "i8", 1, 1), ("bool", "f32", 1, 1.0),
]


@pytest.mark.parametrize("src,dst,v,want", CASES_TO_INT)
def test_checked_cast_boundaries(src, dst, v, want):
    x = np.array([v], O.CARRIERS[src] if src != "bool" else np.uint8)
    y, first, kind = O.cast(src, dst, x)
    if isinstance(want, str):
        assert first == 0 and O.FAILURE_KINDS[kind] == want
        assert O.trap_text(kind, "cast", dst) == f"numeric trap: {want} in cast at {dst}"
    else:
        assert first == -1 and y[0] == want


def test_cast_reports_the_lowest_index_offender():
    x = np.array([1.0, 2.0, 3.0, 1e20, 4.0, 0.5, 1e20], np.float64)
    _, first, kind = O.cast("f64", "i32", x)
    assert (first, O.FAILURE_KINDS[kind]) == (3, "overflow")
    x[2] = np.nan
    _, first, kind = O.cast("f64", "i32", x)
    assert (first, O.FAILURE_KINDS[kind]) == (2, "domain")


# ---------------------------------------------------------------- integer arithmetic
def _wrap(v, bits):
    half = 1 << (bits - 1)
    return (v + half) % (1 << bits) - half


def _py(op, x, y, bits=64):
    if op in ("bitand", "bitor", "bitxor"):
        # Python's integers behave as infinite two's complement
        return x & y if op == "bitand" else x | y if op == "bitor" else x ^ y
    if op in ("shl", "shr"):
        # [05-OP-47] / [04-NUM-13], spec/05-risc-primitives.md:4062-4082
        if y < 0:
            return "domain"
        if op == "shl":
            return 0 if y >= bits else _wrap(x << y, bits)
        return (-1 if x < 0 else 0) if y >= bits else x >> y
    if op == "add":
        return x + y
    if op == "sub":
        return x - y
    if op == "mul":
        return x * y
    if op in ("max_elem", "min_elem"):
        return max(x, y) if op == "max_elem" else min(x, y)
    if y == 0:
        return "division by zero"
    if op == "floor_div":
        return x // y  # Python rounds toward -inf
    if op == "trunc_div":
        q = abs(x) // abs(y)
        return q if (x >= 0) == (y > 0) else -q
    # mod: the remainder of the truncated quotient
    q = abs(x) // abs(y)
    return x - y * (q if (x >= 0) == (y > 0) else -q)


@pytest.mark.parametrize("dt", ["i8", "i16", "i32", "i64"])
@pytest.mark.parametrize("op", list(O.INT_BINARY))
def test_integer_binary_against_unbounded_integers(op, dt):
    info = np.iinfo(CAR[dt])
    rng = np.random.default_rng(len(op) * 7 + info.bits)
    edge = [info.min, info.min + 1, -1, 0, 1, 2, info.max - 1, info.max]
    a = np.concatenate([np.repeat(edge, len(edge)), rng.integers(info.min, info.max, 200, dtype=CAR[dt],
                                                                 endpoint=True)]).astype(CAR[dt])
    b = np.concatenate([np.tile(edge, len(edge)), rng.integers(-4, 5, 100).astype(CAR[dt]),
                        rng.integers(info.min, info.max, 100, dtype=CAR[dt], endpoint=True)]).astype(CAR[dt])
    for i in range(len(a)):
        y, first, kind = O.int_binary(op, dt, a[i:i + 1], b[i:i + 1])
        want = _py(op, int(a[i]), int(b[i]), info.bits)
        if isinstance(want, str):
            assert first == 0 and O.FAILURE_KINDS[kind] == want
        elif want < info.min or want > info.max:
            assert first == 0 and O.FAILURE_KINDS[kind] == "overflow", (op, a[i], b[i])
        else:
            assert first == -1 and int(y[0]) == want, (op, a[i], b[i])


def test_integer_division_known_answers():
    a, b = [7, 7, -7, -7], [2, -2, 2, -2]
    for dt in ("i8", "i16", "i32", "i64"):
        assert O.int_binary("trunc_div", dt, a, b)[0].tolist() == [3, -3, -3, 3]
        assert O.int_binary("floor_div", dt, a, b)[0].tolist() == [3, -4, -4, 3]
        assert O.int_binary("mod", dt, a, b)[0].tolist() == [1, 1, -1, -1]
        lo = int(np.iinfo(CAR[dt]).min)
        _, first, kind = O.int_binary("floor_div", dt, [7], [0])
        assert O.trap_text(kind, "floor_div", dt) == f"numeric trap: division by zero in floor_div at {dt}"
        assert O.int_binary("mod", dt, [lo], [-1])[1:] == (-1, 0)
        assert O.int_binary("mod", dt, [lo + 1], [2])[0].tolist() == [-1]
        assert O.int_binary("trunc_div", dt, [lo], [-1])[2] == 1


def test_integer_trap_texts_of_the_c_lane():
    _, first, kind = O.int_binary("add", "i8", [100, 127], [50, 1])
    assert first == 0 and O.trap_text(kind, "add", "i8") == "numeric trap: overflow in add at i8"
    _, first, kind = O.int_binary("mul", "i8", [1, 64], [1, 2])
    assert first == 1 and O.trap_text(kind, "mul", "i8") == "numeric trap: overflow in mul at i8"
    _, first, kind = O.int_unary("neg", "i64", [5, -(2 ** 63)])
    assert first == 1 and O.trap_text(kind, "neg", "i64") == "numeric trap: overflow in neg at i64"


def test_shift_known_answers():
    """The spec's cases: counts at or above w give 0 (shr of a negative
    value -1), shr extends the sign, shl drops the bits past w."""
    assert O.int_binary("shl", "i8", [1, 1, -1, 3, 64], [7, 8, 1, 100, 1])[0].tolist() == [-128, 0, -2, 0, -128]
    assert O.int_binary("shr", "i8", [-128, -128, -1, 127, -5], [7, 8, 100, 6, 1])[0].tolist() == [-1, -1, -1, 1, -3]
    assert O.int_binary("shr", "i64", [-(2 ** 63), 2 ** 62], [63, 62])[0].tolist() == [-1, 1]
    assert O.int_binary("bitxor", "i16", [-1, 0x5555], [0x00FF, -1])[0].tolist() == [-256, -0x5556]
    y, first, kind = O.int_binary("shl", "i32", [1, 2, 3], [0, -3, -1])
    assert (first, O.FAILURE_KINDS[kind]) == (1, "domain")


@pytest.mark.parametrize("dt", ["i8", "i32", "i64"])
def test_integer_unary(dt):
    info = np.iinfo(CAR[dt])
    x = np.array([info.min + 1, -3, 0, 5, info.max], CAR[dt])
    assert O.int_unary("neg", dt, x)[0].tolist() == [-int(v) for v in x]
    assert O.int_unary("abs", dt, x)[0].tolist() == [abs(int(v)) for v in x]
    assert O.int_unary("abs", dt, np.array([1, info.min], CAR[dt]))[1:] == (1, 1)


# ---------------------------------------------------------------- gather
@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_gather_is_take(itype):
    rng = np.random.default_rng(8)
    v = rng.standard_normal((4, 5, 6))
    for axis in range(3):
        idx = rng.integers(0, v.shape[axis], (3, 2)).astype(itype)
        out, first, _ = O.gather(v, idx, axis)
        assert first == -1
        assert np.array_equal(out, np.take(v, idx, axis=axis))


def test_gather_with_batch_axes_pairs_them():
    rng = np.random.default_rng(9)
    v = rng.standard_normal((3, 7, 2)).astype(np.float32)
    idx = rng.integers(0, 7, (3, 4)).astype(np.int64)
    out, first, _ = O.gather(v, idx, 1, batch_rank=1)
    assert first == -1 and out.shape == (3, 4, 2)
    for bt in range(3):
        assert np.array_equal(out[bt], np.take(v[bt], idx[bt], axis=0))


def test_gather_out_of_range_is_a_domain_trap_at_the_first_index():
    v = np.arange(10.0).reshape(2, 5)
    idx = np.array([1, 5, -1, 2], np.int64)
    out, first, kind = O.gather(v, idx, 1)
    # result [2, 4]: row 0 fails first at its position 1
    assert (first, O.trap_text(kind, "gather", "i64")) == (1, "numeric trap: domain in gather at i64")
    assert out[0, 1] == 0 and out[1, 0] == 6.0


# ---------------------------------------------------------------- extrema cotangent
@pytest.mark.parametrize("dt", ["f32", "f64", "bf16", "f16"])
def test_extrema_adjoint_routes_the_cotangent_to_the_selected_operand(dt):
    """[05-OP-40] in words (spec/05-risc-primitives.md:289-302): the first
    NaN in operand order is selected; otherwise the numerical maximum
    (minimum), the first operand on every equality (signed zeros equal);
    the selected operand gets the whole cotangent, the other +0. The
    selection is read off exact rational order."""
    rng = np.random.default_rng(12)
    v = _values(dt, rng)
    a = np.repeat(v, len(v))
    b = np.tile(v, len(v))
    g = (np.arange(a.size) % 251 + 1).astype(np.float64)
    if dt in ("bf16", "f16"):
        g = O.narrow_encode(dt, g.astype(np.float32))
    else:
        g = g.astype(CAR[dt])
    for kind in ("max", "min"):
        left = O.extrema_adjoint(kind, "left", dt, a, b, g)
        right = O.extrema_adjoint(kind, "right", dt, a, b, g)
        for i in range(a.size):
            na, x = _exact(dt, a[i])
            nb, y = _exact(dt, b[i])
            if na or nb:
                pick_left = na
            else:
                pick_left = (x >= y) if kind == "max" else (x <= y)
            gl, gr = (g[i], 0) if pick_left else (0, g[i])
            assert left.view(np.uint8).reshape(a.size, -1)[i].tobytes() == np.array(
                [gl], g.dtype).view(np.uint8).tobytes(), (kind, dt, a[i], b[i])
            assert right.view(np.uint8).reshape(a.size, -1)[i].tobytes() == np.array(
                [gr], g.dtype).view(np.uint8).tobytes(), (kind, dt, a[i], b[i])


# ---------------------------------------------------------------- ordered scan
def _bf16_rne(f32):
    b = f32.view(np.uint32).astype(np.uint64)
    up = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return up.astype(np.uint16)


@pytest.mark.parametrize("dt", ["f32", "f64", "bf16", "f16"])
@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_floats_are_the_sequential_left_fold(dt, reverse):
    """[05-OP-33]: numpy's add.accumulate (a sequential fold) at the
    accumulator width - binary32 for the 16-bit dtypes, each prefix then
    rounded to nearest even - along either direction; a -0 first leaf stays
    -0 (no base is added)."""
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((5, 300, 7)) * 10.0 ** rng.integers(-3, 4, (5, 300, 7)))
    x[0, 0, 0] = -0.0
    for axis in range(3):
        if dt in ("f32", "f64"):
            xv = x.astype(CAR[dt])
            acc = np.flip(np.cumsum(np.flip(xv, axis), axis, dtype=CAR[dt]), axis) if reverse else np.cumsum(
                xv, axis, dtype=CAR[dt])
            got, first, _ = O.cumsum(dt, xv, axis, reverse)
            want = acc
        else:
            bits = O.narrow_encode(dt, x.astype(np.float32))
            f = O.narrow_decode(dt, bits)
            acc = np.flip(np.cumsum(np.flip(f, axis), axis, dtype=np.float32), axis) if reverse else np.cumsum(
                f, axis, dtype=np.float32)
            want = acc.astype(np.float16).view(np.uint16) if dt == "f16" else _bf16_rne(acc)
            got, first, _ = O.cumsum(dt, bits, axis, reverse)
        assert first == -1
        assert got.tobytes() == want.tobytes(), (dt, axis, reverse)
    got, _, _ = O.cumsum("f32", np.array([-0.0, -0.0], np.float32), 0)
    assert got.view(np.uint32).tolist() == [0x80000000, 0x80000000]
    got, _, _ = O.cumsum("f32", np.array([1.0, np.nan, 2.0], np.float32), 0)
    assert got.view(np.uint32).tolist()[1:] == [0x7FC00000, 0x7FC00000]


@pytest.mark.parametrize("dt", ["i8", "i16", "i32", "i64"])
def test_cumsum_integers_exact_with_the_overflow_trap(dt):
    """Python's unbounded integers; i8 / i16 scan into i32; the first
    overflowing prefix in the evaluation order (line by line)."""
    rng = np.random.default_rng(14)
    info = np.iinfo(CAR[dt])
    x = rng.integers(info.min, info.max, (4, 50, 3), dtype=CAR[dt], endpoint=True)
    if dt in ("i32", "i64"):
        x = (x // 1000).astype(CAR[dt])
    got, first, kind = O.cumsum(dt, x, 1)
    want = np.cumsum(x.astype(object), 1)
    assert first == -1 and got.tolist() == want.tolist()
    assert got.dtype == (np.int32 if dt in ("i8", "i16", "i32") else np.int64)
    if dt in ("i32", "i64"):
        big = np.iinfo(CAR[dt]).max
        y = np.array([[[1], [big], [5]], [[0], [0], [0]]], CAR[dt])  # [2, 3, 1]: line 0 overflows at step 1
        _, first, kind = O.cumsum(dt, y, 1)
        assert (first, O.trap_text(kind, "cumsum", dt)) == (1, f"numeric trap: overflow in cumsum at {dt}")


# ---------------------------------------------------------------- movement with bounds
@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.uint16, np.int8, np.int32, np.int64])
def test_pad_is_numpy_constant_pad(dtype):
    rng = np.random.default_rng(15)
    for shape, pads in [((5, 7), [(1, 2), (0, 3)]), ((3, 1, 4), [(0, 0), (2, 2), (1, 0)]), ((6,), [(4, 0)]),
                        ((2, 0, 3), [(1, 1), (2, 0), (0, 1)])]:
        x = (rng.standard_normal(shape) * 50).astype(dtype)
        fill = dtype(7) if dtype != np.float32 else np.float32(-0.0)
        want = np.pad(x, pads, constant_values=fill)
        got = O.pad(x, [p[0] for p in pads], [p[1] for p in pads], fill)
        assert got.shape == want.shape and got.tobytes() == want.tobytes(), (shape, pads)


def test_shrink_and_stride_are_numpy_slices():
    x = np.arange(5 * 9 * 4, dtype=np.float64).reshape(5, 9, 4) * 1.5
    assert O.slice_(x, [1, 2, 0], [1, 1, 1], [3, 6, 4]).tobytes() == x[1:4, 2:8, :].tobytes()
    for steps in ([1, 2, 3], [2, 4, 1], [5, 9, 4], [7, 1, 2]):
        out = [-(-e // s) for e, s in zip(x.shape, steps)]
        want = x[::steps[0], ::steps[1], ::steps[2]]
        assert O.slice_(x, [0, 0, 0], steps, out).tobytes() == np.ascontiguousarray(want).tobytes(), steps
    assert O.slice_(x, [2, 3, 1], [1, 1, 1], [0, 6, 3]).size == 0


# ---------------------------------------------------------------- scatters
def _destinations(target_shape, idx, axis):
    """Flat target destination of every update (hyperplane form, no batch
    axes): numpy's own index arithmetic over the gathered shape."""
    ushape = target_shape[:axis] + idx.shape + target_shape[axis + 1:]
    coords = list(np.unravel_index(np.arange(int(np.prod(ushape))), ushape))
    k = idx.ndim
    sel = idx[tuple(coords[axis:axis + k])]
    tcoords = coords[:axis] + [sel] + coords[axis + k:]
    return np.ravel_multi_index(tuple(tcoords), target_shape)


@pytest.mark.parametrize("dt", ["f32", "f64", "i16", "i64"])
def test_scatter_replace_keeps_the_highest_position(dt):
    """Last write wins: every targeted cell holds the update whose row-major
    position is the largest among those aimed at it (np.maximum.at over the
    positions), every other cell the target's value."""
    rng = np.random.default_rng(16)
    for shape, axis, ishape in (((6, 9, 4), 1, (5,)), ((7, 3), 0, (4, 2)), ((5, 8), 1, (20,))):
        target = (rng.standard_normal(shape) * 100).astype(CAR[dt])
        idx = rng.integers(0, shape[axis], ishape)
        upd = (rng.standard_normal(O.gather_shape(shape, ishape, axis, 0)) * 100).astype(CAR[dt])
        got, first, _ = O.scatter(dt, target, idx, upd, axis)
        dest = _destinations(shape, idx, axis)
        win = np.full(target.size, -1, np.int64)
        np.maximum.at(win, dest, np.arange(dest.size))
        want = target.reshape(-1).copy()
        hit = win >= 0
        want[hit] = upd.reshape(-1)[win[hit]]
        assert first == -1 and got.reshape(-1).tobytes() == want.tobytes(), (shape, axis)


@pytest.mark.parametrize("dt", ["f32", "f64"])
def test_scatter_add_folds_each_destination_by_the_canonical_tree(dt):
    """Each targeted cell is the canonical tree sum (O.tree_sum, pinned
    with the reductions) of [its target value, its updates in ascending
    position]; with integer-valued operands it is np.add.at exactly."""
    rng = np.random.default_rng(17)
    target = (rng.standard_normal((40, 6)) * 10.0 ** rng.integers(-3, 6, (40, 6))).astype(CAR[dt])
    idx = rng.integers(0, 40, 300)
    upd = (rng.standard_normal((300, 6)) * 10.0 ** rng.integers(-3, 6, (300, 6))).astype(CAR[dt])
    got, first, _ = O.scatter(dt, target, idx, upd, 0, add=True)
    assert first == -1
    for r in range(40):
        rows = np.nonzero(idx == r)[0]
        for c in range(6):
            want = target[r, c] if rows.size == 0 else O.tree_sum(np.concatenate([[target[r, c]], upd[rows, c]]).astype(CAR[dt]))
            assert np.array([got[r, c]]).tobytes() == np.array([want], CAR[dt]).tobytes(), (r, c)
    ti = rng.integers(-50, 50, (40, 6)).astype(CAR[dt])
    ui = rng.integers(-50, 50, (300, 6)).astype(CAR[dt])
    want = ti.copy()
    np.add.at(want, idx, ui)
    assert np.array_equal(O.scatter(dt, ti, idx, ui, 0, add=True)[0], want)


def test_scatter_add_known_answers():
    """bf16 rounds at every node: [256, 1, 1] gives (256 + 1 -> 256) + 1 ->
    256 (each tie to even), where one rounding of the exact 258 keeps 258.
    An i8 tree (100 + 27) + (1 + -1) stays in range where a left fold
    (100 + 27 + 1) would not. A f32 tree [1e8, 4, 4, 4, 4] gives 100000016,
    a left fold 1e8."""
    b = lambda v: O.narrow_encode("bf16", np.array(v, np.float32))
    got, _, _ = O.scatter("bf16", b([256.0, 0.0]), np.array([0, 0]), b([1.0, 1.0]), 0, add=True)
    assert O.narrow_decode("bf16", got).tolist() == [256.0, 0.0]
    got, first, _ = O.scatter("i8", np.array([100], np.int8), np.array([0, 0, 0]), np.array([27, 1, -1], np.int8),
                              0, add=True)
    assert first == -1 and got.tolist() == [127]
    got, first, kind = O.scatter("i8", np.array([100, 0], np.int8), np.array([1, 0, 0]),
                                 np.array([5, 27, 1], np.int8), 0, add=True)
    assert (first, O.trap_text(kind, "scatter", "i8")) == (3 + 0, "numeric trap: overflow in scatter at i8")
    got, _, _ = O.scatter("f32", np.array([1e8], np.float32), np.zeros(4, np.int64), np.full(4, 4.0, np.float32), 0,
                          add=True)
    assert got.tolist() == [100000016.0]


def test_scatter_domain_failure_and_batch_axes():
    target = np.zeros((3, 5), np.float32)
    _, first, kind = O.scatter("f32", target, np.array([1, 4, 5, -1]), np.ones((3, 4), np.float32), 1)
    assert (first, O.FAILURE_KINDS[kind]) == (2, "domain")
    # one batch axis: row b of the target takes row b's own indices
    idx = np.array([[0, 2], [4, 4], [1, 0]])
    upd = np.arange(6, dtype=np.float32).reshape(3, 2) + 1
    got, first, _ = O.scatter("f32", target, idx, upd, 1, batch_rank=1, add=True)
    want = np.zeros((3, 5), np.float32)
    for r in range(3):
        for j in range(2):
            want[r, idx[r, j]] += upd[r, j]
    assert first == -1 and np.array_equal(got, want)


@pytest.mark.parametrize("dt", ["f32", "i32"])
def test_scatter_elements_keeps_the_highest_position(dt):
    rng = np.random.default_rng(18)
    data = (rng.standard_normal((6, 7, 5)) * 100).astype(CAR[dt])
    for axis in range(3):
        ishape = (4, 3, 5) if axis != 2 else (6, 7, 9)
        idx = rng.integers(0, data.shape[axis], ishape)
        upd = (rng.standard_normal(ishape) * 100).astype(CAR[dt])
        got, first, _ = O.scatter_elements(dt, data, idx, upd, axis)
        coords = list(np.unravel_index(np.arange(idx.size), ishape))
        coords[axis] = idx.reshape(-1)
        dest = np.ravel_multi_index(tuple(coords), data.shape)
        win = np.full(data.size, -1, np.int64)
        np.maximum.at(win, dest, np.arange(dest.size))
        want = data.reshape(-1).copy()
        want[win >= 0] = upd.reshape(-1)[win[win >= 0]]
        assert first == -1 and got.reshape(-1).tobytes() == want.tobytes(), axis
    bad = np.zeros((6, 7, 5), np.int64)
    bad[1, 2, 3] = 7
    assert O.scatter_elements(dt, data, bad, np.zeros((6, 7, 5), CAR[dt]), 2)[1] == (1 * 7 + 2) * 5 + 3

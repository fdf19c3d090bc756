"""Pins of the CPU oracle against the reference's own golden vectors, an
independent restatement or what the mathematics fixes. CPU only.

What pins what:
  RNG (splitmix64/derive/word/unit/split/fold_in/split_n): KAT hex values of
      crates/chelis-numeric-core/tests/random_key_reference.rs:86-140.
  keyed dropout + replay: crates/chelis-cli/tests/dropout_fixed_stream_cli.rs
      (fixed-stream vectors [2,0,0,2] and [2,2,0,0]).
  correctly rounded exp/log/erfc/tanh: CORE-MATH MPFR canary fixture
      (crates/chelis-crmath/tests/fixtures/canary.txt), bit for bit.
  canonical tree sum: the pass-by-pass restatement of spec/05 section 2.3 in
      C and an independent numpy restatement, on inputs whose bits change
      under any other association; the [05-OP-30] trace (((a+b)+(c+d))+e).
  max_reduce: the first-NaN and first-representation rules of [05-OP-12].
  matmul: crates/chelis-cli/tests/fixtures/inlined_product/matmul.expected;
      lanes vs the scalar tree on random shapes.
  softmax / layer norm / GELU: float64 closed forms within a few ulps plus
      special values fixed by the spec (GELU(-inf) = -0, Phi graph limits).
"""
import json
import math
from fractions import Fraction
import os
import struct

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def setup_module(_m):
    O.build()


def h(s):
    return int(s, 16)


# ---------------------------------------------------------------- RNG
def test_rng_known_answers():
    g = json.load(open(os.path.join(GOLD, "key_reference.json")))
    k7 = 7
    assert O.split(k7) == tuple(h(v) for v in g["key7_split"])
    assert O.fold_in(k7, 3) == h(g["key7_fold_in_3"])
    assert O.fold_in(k7, -1) == h(g["key7_fold_in_minus1"])
    assert O.split_n(k7, 3) == [h(v) for v in g["key7_split_n_3"]]
    assert int(O.lib().orc_derive(k7, 2)) == h(g["key7_derive_2"])
    assert O.unit(k7, 0) == g["key7_units_1"][0]
    c = g["chain"]
    km3 = (-3) & (2**64 - 1)
    assert km3 == h(c["key_minus3_bits"])
    left, right = O.split(km3)
    assert (left, right) == (h(c["split_left"]), h(c["split_right"]))
    folded = O.fold_in(left, -5)
    assert folded == h(c["left_fold_in_minus5"])
    assert O.split_n(folded, 3) == [h(v) for v in c["folded_split_n_3"]]
    assert O.fold_in(right, 9) == h(c["right_fold_in_9"])


def test_dropout_fixed_stream():
    g = json.load(open(os.path.join(GOLD, "key_reference.json")))["dropout_fixed_stream"]
    left, right = O.split(g["seed"])
    x = np.array(g["x"], np.float32)
    assert O.dropout(right, x, np.float32(g["rate"])).tolist() == g["forward_right_key"]
    # grad of sum(dropout(left, x)) wrt x is the replay of ones
    assert O.dropout_replay(left, np.ones(4, np.float32), np.float32(g["rate"])).tolist() == g["grad_left_key"]
    # at binary64 the same stream: the unit at 53 bits against the rate
    assert O.dropout_replay(left, np.ones(4, np.float64), g["rate"]).tolist() == g["grad_left_key"]
    assert O.dropout(right, x.astype(np.float64), g["rate"]).tolist() == g["forward_right_key"]


def test_dropout_rate_zero_is_identity_and_mask_matches_units():
    key = O.fold_in(44, 0)
    x = np.random.default_rng(0).standard_normal(4096).astype(np.float32)
    assert np.array_equal(O.dropout(key, x, np.float32(0.0)), x)
    y = O.dropout(key, x, np.float32(0.1))
    units = np.array([O.unit(key, i) for i in range(x.size)])
    dropped = units.astype(np.float32) < np.float32(0.1)
    assert np.array_equal(y == 0, dropped | (x == 0))
    assert np.array_equal(y[~dropped], x[~dropped] / (np.float32(1) - np.float32(0.1)))
    assert 0.08 < dropped.mean() < 0.12


def test_uniform_like_is_the_fma_of_the_unit():
    key = 12345
    u = O.uniform_like(key, np.float64(0.0), np.float64(1.0), 64, np.float64)
    assert [O.unit(key, i) for i in range(64)] == u.tolist()


def _round_f32(q: Fraction) -> np.float32:
    """The binary32 value nearest the exact rational q, ties to even (finite
    range only): one rounding, independent of numpy's float arithmetic."""
    c = np.float32(float(q))  # within one binary32 ulp of q
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(cand)) - q)
        key = (d, int(np.array(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return best[1]


def test_uniform_like_f32_is_one_rounding_of_the_exact_affine_map():
    """[05-OP-8] at f32: fmaf(high - low, (float)unit, low). Against the exact
    rational span * u32 + low rounded once; a multiply-then-add (two
    roundings) differs on many of these elements, so the check has teeth."""
    key, n = O.fold_in(77, 5), 4096
    low, high = np.float32(-1.5), np.float32(2.25)
    span = high - low  # 3.75, exact
    got = O.uniform_like(key, low, high, n, np.float32)
    two_roundings = 0
    for i in range(n):
        u32 = np.float32(O.unit(key, i))
        exact = Fraction(float(span)) * Fraction(float(u32)) + Fraction(float(low))
        want = _round_f32(exact)
        assert got[i].view(np.uint32) == np.array(want).view(np.uint32), i
        two_roundings += (span * u32 + low) != want
    assert two_roundings > 50


def test_uniform_like_f64_is_one_rounding_of_the_exact_affine_map():
    """[05-OP-8] at f64: fma(high - low, unit, low), against the exact rational
    rounded once (Python's int / int division is correctly rounded)."""
    key, n = O.fold_in(78, 1), 4096
    low, high = -0.7, 2.9  # span 3.5999999999999996: products round
    span = np.float64(high) - np.float64(low)
    got = O.uniform_like(key, np.float64(low), np.float64(high), n, np.float64)
    two_roundings = 0
    for i in range(n):
        u = O.unit(key, i)
        exact = Fraction(float(span)) * Fraction(u) + Fraction(low)
        want = float(exact)
        assert got[i] == want and np.signbit(got[i]) == np.signbit(want), i
        two_roundings += float(span) * u + low != want
    assert two_roundings > 50


def test_dropout_f64_mask_is_the_binary64_unit_and_kept_values_are_one_division():
    """[05-OP-37] at f64 (crates/chelis-backend-c/src/emit.rs:6179-6189): the
    binary64 unit is compared with the binary64 rate (no binary32 rounding of
    the unit), a kept element is x / (1 - rate) rounded once. Element 7's
    rate is placed between its unit and that unit's binary32 rounding, so a
    binary32 comparison would keep an element the binary64 rule drops."""
    key, n = O.fold_in(91, 3), 2048
    x = np.random.default_rng(5).standard_normal(n) * 10.0 ** np.random.default_rng(6).integers(-30, 30, n)
    u7 = O.unit(key, 7)
    f7 = float(np.float32(u7))
    if f7 < u7:  # make the binary32 rounding of u7 lie above it
        u7 = O.unit(key, 8)
        f7 = float(np.float32(u7))
    assert f7 > u7
    rate = float(Fraction(u7) + (Fraction(f7) - Fraction(u7)) / 2)
    assert u7 < rate < f7
    y = O.dropout(key, x, rate)
    denom = 1.0 - rate
    dropped = 0
    for i in range(n):
        u = O.unit(key, i)
        if u < rate:
            assert y[i] == 0.0 and not np.signbit(y[i]), i
            dropped += 1
        else:
            assert y[i] == float(Fraction(float(x[i])) / Fraction(denom)), i
    kept32 = [i for i in range(n) if not (np.float32(O.unit(key, i)) < np.float32(rate))]
    assert y[[i for i in kept32 if O.unit(key, i) < rate]].tolist() != []
    assert 0 < dropped < n


# ---------------------------------------------------------------- prod
def test_prod_axis_is_the_left_fold_of_the_c_lane():
    """ProdReduce = ((1 * x0) * x1) * x2 ... at the dtype
    (crates/chelis-backend-c/src/emit.rs:2551-2561). Hand-derived answers
    that any other association or a dropped factor changes:
      [1e-30, 1e-30, 1e30, 1e30] f32: 1e-60 underflows to +0, so the fold is
        +0; pairwise (1e-60 -> 0) * (1e60 -> inf) is NaN.
      [2^100, 2^100, 2^-100, 2^-100] f32: the fold overflows to inf at the
        second factor and stays inf; pairwise it is exactly 1.
      [3, 5, 7, 11] and powers of two: exact products.
      a NaN anywhere: the canonical quiet NaN.
      an empty axis: 1 (the identity, no multiply)."""
    f = np.float32
    def run(v, dt=np.float32):
        return O.prod_axis(np.array([v], dt), 1)[0]
    assert run([1e-30, 1e-30, 1e30, 1e30]) == 0.0
    assert run([2.0 ** 100, 2.0 ** 100, 2.0 ** -100, 2.0 ** -100]) == np.inf
    assert run([3, 5, 7, 11]) == f(1155)
    assert run([0.5, -4, 0.25, 2]) == f(-1)
    nan = run([1, float("nan"), 2])
    assert np.array(nan).view(np.uint32) == 0x7FC00000
    assert O.prod_axis(np.zeros((3, 0), np.float32), 1).tolist() == [1.0, 1.0, 1.0]
    # binary64: 1e-200 * 1e-200 underflows to +0 before the 1e200 factors
    assert run([1e-200, 1e-200, 1e200, 1e200], np.float64) == 0.0
    # left-to-right rounding: for these three binary32 values (bits below)
    # ((1 * a) * b) * c rounds to 0x4057ed10 while a * (b * c) rounds to
    # 0x4057ed0f (each product taken exactly as a rational and rounded once
    # with _round_f32)
    a, b, c = np.array([0x3FC1835F, 0x3FF9A8CB, 0x3F9273D2], np.uint32).view(np.float32)
    F = lambda v: Fraction(float(v))
    left = _round_f32(F(_round_f32(F(a) * F(b))) * F(c))
    right = _round_f32(F(a) * F(_round_f32(F(b) * F(c))))
    assert np.array(left).view(np.uint32) == 0x4057ED10 and np.array(right).view(np.uint32) == 0x4057ED0F
    assert np.array(run([a, b, c])).view(np.uint32) == 0x4057ED10
    # axis 0 of a [n, m] matrix folds each column top to bottom
    m = np.array([[2, 3], [5, 7], [11, 13]], np.float32)
    assert O.prod_axis(m, 0).tolist() == [110.0, 273.0]


# ---------------------------------------------------------------- CORE-MATH
def _canary_rows():
    rows = []
    for line in open(os.path.join(GOLD, "crmath_canary.txt")):
        if line.startswith("#") or not line.strip():
            continue
        fn, width, xin, xout = line.split()[:4]
        rows.append((fn, width, xin, xout))
    return rows


@pytest.mark.parametrize("fn", ["exp", "log", "erfc", "tanh"])
def test_correctly_rounded_leaves_match_mpfr_canary(fn):
    L = O.lib()
    n = 0
    for f, width, xin, xout in _canary_rows():
        if f != fn:
            continue
        if width == "f32":
            x = struct.unpack("<f", struct.pack("<I", h(xin)))[0]
            got = struct.unpack("<I", struct.pack("<f", getattr(L, f"orc_{fn}f")(x)))[0]
        else:
            x = struct.unpack("<d", struct.pack("<Q", h(xin)))[0]
            got = struct.unpack("<Q", struct.pack("<d", getattr(L, f"orc_{fn}")(x)))[0]
        assert got == h(xout), (fn, width, xin)
        n += 1
    assert n > 30


# ---------------------------------------------------------------- tree sum
def _np_level_sum(x):
    """Independent numpy restatement of spec/05 section 2.3's level passes."""
    vals = list(x)
    if not vals:
        return x.dtype.type(0)
    while len(vals) > 1:
        nxt = [vals[i] + vals[i + 1] for i in range(0, len(vals) - 1, 2)]
        if len(vals) % 2:
            nxt.append(vals[-1])
        vals = nxt
    return vals[0]


def _adversarial(n, dtype, seed):
    rng = np.random.default_rng(seed)
    mag = rng.choice([1e-8, 1.0, 1e8, 3e-3], size=n)
    return (rng.standard_normal(n) * mag).astype(dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_tree_sum_matches_level_passes(dtype):
    ns = list(range(0, 70)) + [2**k + d for k in range(6, 13) for d in (-1, 0, 1)] + [1000, 4095]
    for n in ns:
        x = _adversarial(n, dtype, n)
        t = O.tree_sum(x)
        assert t.tobytes() == O.level_sum(x).tobytes(), n
        if n <= 300:
            assert t.tobytes() == dtype(_np_level_sum(x)).tobytes(), n


def test_tree_sum_shape_is_the_canonical_trace():
    # (((a+b)+(c+d))+e): with a=1e8, c=-1e8 the pairwise sums keep b,d exact
    # only under this association.
    x = np.array([1e8, 1.0, -1e8, 1.0, 0.5], np.float32)
    a, b, c, d, e = (np.float32(v) for v in x)
    assert O.tree_sum(x) == ((a + b) + (c + d)) + e
    assert O.tree_sum(x) != (((a + b) + c) + d) + e   # a left fold differs


def test_tree_sum_empty_and_signed_zero():
    assert O.tree_sum(np.zeros(0, np.float32)).tobytes() == np.float32(0).tobytes()
    assert O.tree_sum(np.array([-0.0], np.float32)).tobytes() == np.float32(-0.0).tobytes()
    assert O.tree_sum(np.array([-0.0, -0.0, -0.0], np.float64)).tobytes() == np.float64(-0.0).tobytes()
    nan = O.tree_sum(np.array([1.0, np.inf, -np.inf], np.float32))
    assert nan.view(np.uint32) == 0x7FC00000


def test_sum_axis_is_tree_per_slice():
    x = _adversarial(5 * 37 * 3, np.float32, 1).reshape(5, 37, 3)
    s = O.sum_axis(x, 1)
    for o in range(5):
        for j in range(3):
            assert s[o, j] == O.tree_sum(x[o, :, j].copy())


# ---------------------------------------------------------------- max / count
def test_max_reduce_first_nan_and_first_representation():
    nan_a = np.array([0x7FC00001], np.uint32).view(np.float32)[0]
    nan_b = np.array([0xFFC00002], np.uint32).view(np.float32)[0]
    x = np.array([1.0, nan_a, 5.0, nan_b], np.float32)
    assert O.max_axis(x, 0).view(np.uint32) == 0x7FC00001
    z = np.array([-0.0, 0.0, -1.0], np.float32)
    assert O.max_axis(z, 0).tobytes() == np.float32(-0.0).tobytes()
    r = np.random.default_rng(3).standard_normal((64, 33))
    assert np.array_equal(O.max_axis(r, 1), r.max(1))


def test_count_axis():
    rng = np.random.default_rng(4)
    b = (rng.random((7, 300)) < 0.3).astype(np.uint8)
    c, err = O.count_axis(b, 1)
    assert err == 0 and np.array_equal(c, b.sum(1))
    b[3, 5] = 2
    assert O.count_axis(b, 1)[1] == 1


# ---------------------------------------------------------------- matmul
def _decimal(v):
    if np.isnan(v):
        return "NaN"
    if np.isinf(v):
        return "inf" if v > 0 else "-inf"
    r = repr(float(v)) if v.dtype == np.float64 else str(v)
    return r.replace("e+", "e")


def test_matmul_inlined_product_golden():
    g = json.load(open(os.path.join(GOLD, "matmul_inlined_product.json")))
    a = np.array(g["a32"], np.float32)
    b = np.array(g["b32"], np.float32)
    c = O.matmul(a, b).ravel()
    assert [_decimal(v) for v in c] == g["f32"]
    c64 = O.matmul(a.astype(np.float64), b.astype(np.float64)).ravel()
    assert [_decimal(v) for v in c64] == g["f64_of_f32_inputs"]
    cr = O.matmul(O.relu(a), b).ravel()
    assert [_decimal(v) for v in cr] == g["relu_a32_f32"]
    ir = O.matmul(np.array(g["inf_row"], np.float32), np.array(g["zero_col"], np.float32)).ravel()
    assert [_decimal(v) for v in ir] == g["inf_row_times_zero_col"]
    sq = O.matmul(a, a.T).ravel()    # strided view: the transpose is not copied
    assert [_decimal(v) for v in sq] == g["square_a32_a32T"]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_matmul_lanes_equal_scalar_tree(dtype):
    rng = np.random.default_rng(5)
    for M, N, K in [(1, 1, 1), (3, 9, 5), (7, 17, 33), (5, 3, 64), (9, 12, 100)]:
        a = _adversarial(M * K, dtype, M).reshape(M, K)
        b = _adversarial(K * N, dtype, N).reshape(K, N)
        c = O.matmul(a, b)
        for i in range(M):
            for j in range(N):
                assert c[i, j].tobytes() == O.tree_sum((a[i] * b[:, j]).astype(dtype)).tobytes()
        ref = a.astype(np.float64) @ b.astype(np.float64)
        assert np.allclose(c, ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())
    del rng


# ---------------------------------------------------------------- row regions
@pytest.mark.parametrize("dtype,n", [(np.float32, 1024), (np.float32, 10), (np.float64, 777)])
def test_softmax_rows_closed_form(dtype, n):
    x = (np.random.default_rng(6).standard_normal((64, n)) * 2).astype(dtype)
    y = O.softmax_rows(x)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(1, keepdims=True))
    ref = e / e.sum(1, keepdims=True)
    # the f32 subtraction x - max rounds at |x - max| * 2^-24 before exp
    tol = 2e-6 if dtype == np.float32 else 1e-14
    assert np.max(np.abs(y - ref) / ref) < tol


def test_softmax_special_rows():
    x = np.array([[0.0, -np.inf, 1.0, -np.inf], [-np.inf] * 4, [3.0, 3.0, 3.0, 3.0], [1.0, np.nan, 0, 0]],
                 np.float32)
    y = O.softmax_rows(x)
    assert y[0, 1] == 0 and y[0, 3] == 0 and abs(y[0].sum() - 1) < 1e-6
    assert (y[1].view(np.uint32) == 0x7FC00000).all()
    assert (y[2] == 0.25).all()
    assert (y[3].view(np.uint32) == 0x7FC00000).all()
    assert O.softmax_rows(np.array([[5.0]], np.float32))[0, 0] == 1.0


def test_layer_norm_closed_form():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((32, 1024)).astype(np.float32)
    g = rng.standard_normal(1024).astype(np.float32)
    b = rng.standard_normal(1024).astype(np.float32)
    y = O.layer_norm_rows(x, g, b, np.float32(1e-5))
    x64 = x.astype(np.float64)
    m = x64.mean(1, keepdims=True)
    v = ((x64 - m) ** 2).mean(1, keepdims=True)
    ref = (x64 - m) / np.sqrt(v + 1e-5) * g + b
    assert np.max(np.abs(y - ref)) < 2e-5


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_gelu_closed_form_and_limits(dtype):
    x = np.concatenate([np.linspace(-12, 12, 20001), np.random.default_rng(8).standard_normal(5000) * 3]).astype(dtype)
    y = O.gelu(x)
    ref = np.array([float(v) * 0.5 * math.erfc(-float(v) / math.sqrt(2)) for v in x])
    big = np.abs(ref) > 1e-30
    rel = np.abs(y[big] - ref[big]) / np.abs(ref[big])
    # the float64 check rounds -x/sqrt(2) before erfc, an argument error the
    # Phi graph corrects; at |x| ~ 12 that costs ~2 t^2 eps ~ 3e-14 relative
    assert rel.max() < (6e-7 if dtype == np.float32 else 5e-14)
    special = O.gelu(np.array([-np.inf, np.inf, 0.0, -0.0, np.nan, -100.0], dtype))
    assert special[0] == 0 and np.signbit(special[0])
    assert special[1] == np.inf and special[2] == 0 and special[3] == 0
    assert np.isnan(special[4]) and special[5] == 0 and np.signbit(special[5])


def test_relu_bit_rules():
    nan_p = np.array([0x7FC01234], np.uint32).view(np.float32)[0]
    x = np.array([-1.0, -0.0, 0.0, 2.0, nan_p], np.float32)
    y = O.relu(x)
    assert y.view(np.uint32).tolist() == [0, 0x80000000, 0, np.float32(2.0).view(np.uint32), 0x7FC01234]
    g = np.full(5, 3.0, np.float32)
    assert O.relu_adjoint(x, g).tolist() == [0, 0, 0, 3.0, 0]


# ---- bfloat16 / binary16 storage ----
def _f32_edge_patterns(rng, n):
    """Random binary32 bit patterns plus every binary16 value's rounding
    midpoint (as binary32) and its two binary32 neighbours."""
    r = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    h = np.arange(0x7c00, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32).view(np.uint32)  # exact: 12 significant bits
    both = np.concatenate([mids, mids - 1, mids + 1])
    return np.concatenate([r, both, both | np.uint32(0x80000000)])


def test_f16_decode_every_pattern_is_ieee():
    h = np.arange(2**16, dtype=np.uint16)
    got = O.narrow_decode("f16", h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_encode_is_ieee_round_to_nearest_even():
    """Against numpy's binary32 -> binary16 conversion (IEEE round to
    nearest even, gradual underflow, overflow to infinity), including every
    binary16 midpoint; NaN is the canonical 0x7e00."""
    x = _f32_edge_patterns(np.random.default_rng(21), 1 << 21).view(np.float32)
    got = O.narrow_encode("f16", x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.all(got[nan] == 0x7E00)
    bad = np.nonzero(got[~nan] != want[~nan])[0]
    assert bad.size == 0, [(hex(int(x[~nan].view(np.uint32)[i])), hex(int(got[~nan][i])), hex(int(want[~nan][i])))
                           for i in bad[:5]]


def test_bf16_encode_is_nearest_even_by_distance():
    """bf16 rounding from its definition: of the two bf16 values around x
    (truncation and the next one away from zero, 2^128 standing for the
    overflow), the nearer by exact binary64 distance, ties to the even
    pattern; NaN is the canonical 0x7fc0."""
    x = np.random.default_rng(22).integers(0, 2**32, 1 << 21, dtype=np.uint64).astype(np.uint32)
    half_ulps = np.arange(0, 2**16, dtype=np.uint32) << 16 | np.uint32(0x8000)  # every exact tie
    x = np.concatenate([x, half_ulps, half_ulps + 1, half_ulps - 1]).view(np.float32)
    got = O.narrow_encode("bf16", x)
    fin = np.isfinite(x)
    assert np.all(got[np.isnan(x)] == 0x7FC0)
    inf = np.isinf(x)
    assert np.array_equal(got[inf], (x[inf].view(np.uint32) >> 16).astype(np.uint16))
    xb = x[fin].view(np.uint32)
    v = x[fin].astype(np.float64)
    lo = (xb & np.uint32(0xFFFF0000)).view(np.float32).astype(np.float64)
    hib = (xb & np.uint32(0xFFFF0000)) + np.uint32(0x10000)
    hi = hib.view(np.float32).astype(np.float64)
    hi = np.where(np.isinf(hi), np.sign(v) * 2.0**128, hi)
    dl, dh = np.abs(v - lo), np.abs(hi - v)
    lo_bits = (xb >> 16).astype(np.uint16)
    want = np.where(dl < dh, lo_bits, lo_bits + 1)
    tie = dl == dh
    want = np.where(tie, np.where(lo_bits & 1, lo_bits + 1, lo_bits), want).astype(np.uint16)
    assert np.array_equal(got[fin], want)


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_narrow_sub_is_binary32_then_one_rounding(kind):
    rng = np.random.default_rng(23)
    a = O.narrow_encode(kind, (rng.standard_normal(100000) * 8).astype(np.float32))
    b = O.narrow_encode(kind, (rng.standard_normal(100000) * 8).astype(np.float32))
    got = O.narrow_binary("sub", kind, a, b)
    diff = (O.narrow_decode(kind, a) - O.narrow_decode(kind, b)).astype(np.float32)
    if kind == "f16":
        want = diff.astype(np.float16).view(np.uint16)  # IEEE narrowing, independent of the oracle's
    else:
        want = O.narrow_encode(kind, diff)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_narrow_selection_special_cases(kind):
    nan1, nan2 = (0x7FC1, 0xFFC3) if kind == "bf16" else (0x7E01, 0xFE03)
    one = 0x3F80 if kind == "bf16" else 0x3C00
    two = 0x4000 if kind == "bf16" else 0x4000
    a = np.array([nan1, one, 0x0000, 0x8000, one, nan1, two], np.uint16)
    b = np.array([one, nan2, 0x8000, 0x0000, two, nan2, one], np.uint16)
    mx = O.narrow_binary("max", kind, a, b)
    mn = O.narrow_binary("min", kind, a, b)
    # NaN on the left wins with its own bits; NaN on the right wins when the
    # left is a number; ties (+0 / -0) keep the left operand
    assert list(mx) == [nan1, nan2, 0x0000, 0x8000, two, nan1, two]
    assert list(mn) == [nan1, nan2, 0x0000, 0x8000, one, nan1, one]


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_narrow_relu_bit_rules(kind):
    nan = 0x7FC1 if kind == "bf16" else 0x7E01
    x = np.array([0x3F80, 0xBF80, 0x0000, 0x8000, nan, nan | 0x8000, 0x0001, 0x8001], np.uint16)
    g = np.full(x.shape, 0x1234, np.uint16)
    assert list(O.narrow_relu(kind, x)) == [0x3F80, 0, 0, 0x8000, nan, nan | 0x8000, 0x0001, 0]
    assert list(O.narrow_relu_adjoint(kind, x, g)) == [0x1234, 0, 0, 0, 0, 0, 0x1234, 0]


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_narrow_matmul_against_float64(kind):
    """decode, binary32 tree product, encode: within one 16-bit rounding of
    the float64 product of the decoded operands; exact on an identity."""
    rng = np.random.default_rng(24)
    a = O.narrow_encode(kind, rng.standard_normal((37, 70)).astype(np.float32))
    b = O.narrow_encode(kind, rng.standard_normal((70, 29)).astype(np.float32))
    c = O.narrow_decode(kind, O.narrow_matmul(kind, a, b)).astype(np.float64)
    ref = O.narrow_decode(kind, a).astype(np.float64) @ O.narrow_decode(kind, b).astype(np.float64)
    ulp = 2.0**-8 if kind == "bf16" else 2.0**-11
    assert np.all(np.abs(c - ref) <= ulp * np.abs(ref) + 1e-5 * np.abs(ref).max())
    eye = O.narrow_encode(kind, np.eye(70, dtype=np.float32))
    assert np.array_equal(O.narrow_matmul(kind, a, eye), a)

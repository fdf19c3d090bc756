"""GPU parity of the row and elementwise regions against the CPU oracle.

Bar: bit-exact where the oracle's leaves are IEEE operations or correctly
rounded transcendentals (softmax f32, layer norm, relu, dropout,
uniform_like, GELU f32, the f32 exp/log/erfc/tanh chain leaves, whose device
results equal CORE-MATH on every binary32 input, the f64 exp leaf, a
correctly rounded binary64 exp, and softmax f64 in the exact mode); 1e-12
relative for f64 GELU, whose device erfc leaf is within an ulp instead of
correctly rounded. The default binary64 softmax row (faithful exp, one
reciprocal per row) is held to 1e-13 relative per element, the same NaN
positions and the canonical NaN bits; the north star's bar for binary64
reductions is 1e-10.
"""
import contextlib

import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def setup_module(_m):
    O.build()


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


@contextlib.contextmanager
def exact_mode(on=True):
    prev = C.set_exact(on)
    try:
        yield
    finally:
        C.set_exact(prev)


def assert_f64_rows_close(y, ref):
    """The default binary64 softmax row against the exact one: NaNs in the
    same places with the same bits, every other element within 1e-13
    relative (plus four units of the least subnormal), row sums within
    1e-12 of the exact row's."""
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(y), nan)
    assert bits_equal(y[nan], ref[nan])
    yf, rf = y[~nan], ref[~nan]
    err = np.abs(yf - rf) - (1e-13 * np.abs(rf) + 4 * 2.0 ** -1074)
    assert (err <= 0).all(), f"max rel {float((np.abs(yf - rf) / np.maximum(np.abs(rf), 1e-300)).max()):.3e}"
    fin = ~nan.any(axis=-1)
    assert np.abs(y[fin].sum(-1) - ref[fin].sum(-1)).max(initial=0.0) <= 1e-12


def mismatch_report(a, b):
    ai = np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint64)
    bi = np.ascontiguousarray(b).view(np.uint32 if b.dtype == np.float32 else np.uint64)
    bad = np.nonzero(ai != bi)
    return f"{len(bad[0])} mismatches; first at {tuple(i[0] for i in bad) if len(bad[0]) else None}"


@pytest.mark.parametrize("n", [1, 3, 10, 64, 100, 255, 256, 257, 512, 1000, 1024, 2048, 2049, 4096, 5000, 16384])
def test_softmax_f32_bit_exact(n):
    rows = max(1, 65536 // n)
    x = (np.random.default_rng(n).standard_normal((rows, n)) * 2).astype(np.float32)
    y = C.softmax(C.to_device(x)).numpy()
    ref = O.softmax_rows(x)
    assert bits_equal(y, ref), mismatch_report(y, ref)


def test_softmax_f32_config_shape_bit_exact():
    """Config 2: [16384, 1024] ~ N(0, sigma=2), compared elementwise and by row sum."""
    x = (np.random.default_rng(10).standard_normal((16384, 1024)) * 2).astype(np.float32)
    y = C.softmax(C.to_device(x)).numpy()
    ref = O.softmax_rows(x)
    assert bits_equal(y, ref), mismatch_report(y, ref)
    assert np.abs(y.astype(np.float64).sum(1) - 1).max() < 1e-5


@pytest.mark.parametrize("exact", [True, False])
def test_softmax_f64_config_shape(exact):
    """Config 2 f64: [4096, 4096] ~ N(0,1); bit-exact in the exact mode
    (correctly rounded binary64 exp, IEEE division), within 1e-13 per
    element in the default mode; and by row sum."""
    x = np.random.default_rng(11).standard_normal((4096, 4096))
    with exact_mode(exact):
        y = C.softmax(C.to_device(x)).numpy()
    ref = O.softmax_rows(x)
    if exact:
        assert bits_equal(y, ref), mismatch_report(y, ref)
    else:
        assert_f64_rows_close(y, ref)
    assert np.abs(y.sum(1) - 1).max() < 1e-10


@pytest.mark.parametrize("n", [1, 5, 100, 256, 1000, 1025, 4096, 5000])
def test_softmax_f64_bit_exact(n):
    rows = max(1, 65536 // n)
    x = np.random.default_rng(100 + n).standard_normal((rows, n)) * 3
    ref = O.softmax_rows(x)
    with exact_mode():
        y = C.softmax(C.to_device(x)).numpy()
    assert bits_equal(y, ref), mismatch_report(y, ref)
    assert_f64_rows_close(C.softmax(C.to_device(x)).numpy(), ref)


def test_softmax_f64_tiny_and_subnormal_quotients():
    """Elements whose exp is below 2^-960 or subnormal take the full division;
    the rest divide by the row reciprocal's steps: both bit-exact in the
    exact mode; the default row within tolerance, subnormals included."""
    rng = np.random.default_rng(99)
    x = rng.uniform(-745.0, 0.0, (256, 4096))
    x[:, 0] = 0.0
    x[::2, 1:64] = rng.uniform(-3.0, 0.0, (128, 63))
    ref = O.softmax_rows(x)
    with exact_mode():
        y = C.softmax(C.to_device(x)).numpy()
    assert bits_equal(y, ref), mismatch_report(y, ref)
    assert_f64_rows_close(C.softmax(C.to_device(x)).numpy(), ref)


@pytest.mark.parametrize("exact", [True, False])
def test_softmax_f64_special_rows(exact):
    """-inf, all -inf (NaN total), NaN, +inf, signed zeros and subnormal
    exps; the NaN rows are canonical NaNs in both modes."""
    x = np.array([[0.0, -np.inf, 1.0, -np.inf], [-np.inf] * 4, [3.0] * 4, [1.0, np.nan, 0, 0],
                  [np.inf, 0, 0, 0], [-0.0, 0.0, -0.0, 0.0], [0.0, -745.0, -708.5, -1e-300]])
    with exact_mode(exact):
        y = C.softmax(C.to_device(x)).numpy()
    ref = O.softmax_rows(x)
    if exact:
        assert bits_equal(y, ref)
    else:
        assert_f64_rows_close(y, ref)
        assert bits_equal(y[1:3], ref[1:3]) and bits_equal(y[5], ref[5])


def test_softmax_special_rows():
    x = np.array([[0.0, -np.inf, 1.0, -np.inf], [-np.inf] * 4, [3.0] * 4, [1.0, np.nan, 0, 0],
                  [np.inf, 0, 0, 0], [-0.0, 0.0, -0.0, 0.0]], np.float32)
    y = C.softmax(C.to_device(x)).numpy()
    assert bits_equal(y, O.softmax_rows(x))


def test_softmax_strided_rows():
    """Rows with a leading stride larger than the row (a column slice)."""
    big = (np.random.default_rng(3).standard_normal((64, 1536)) * 3).astype(np.float32)
    d = C.to_device(big)
    v = d.view((64, 1000), (1536, 1), offset_elems=8)
    out = C.empty((64, 1000), np.float32)
    C.softmax(v, out)
    assert bits_equal(out.numpy(), O.softmax_rows(big[:, 8:1008].copy()))


@pytest.mark.parametrize("causal", [True, False])
def test_scaled_masked_softmax(causal):
    s = 128
    x = np.random.default_rng(5).standard_normal((2, 3, s, s)).astype(np.float32)
    scale = np.float32(0.125)
    y = C.scaled_masked_softmax(C.to_device(x), 0.125, causal).numpy()
    sc = x * scale
    if causal:
        mask = np.tril(np.ones((s, s), bool))
        sc = np.where(mask, sc, np.float32(-np.inf)).astype(np.float32)
    ref = O.softmax_rows(sc.reshape(-1, s)).reshape(x.shape)
    assert bits_equal(y, ref), mismatch_report(y, ref)


@pytest.mark.parametrize("dtype,s", [(np.float32, 512), (np.float64, 512), (np.float32, 100), (np.float64, 37)])
def test_causal_softmax_ignores_the_masked_triangle(dtype, s):
    """Causal rows read only j <= i: NaN and inf planted above the diagonal
    (where the scores product leaves memory unwritten) change nothing."""
    rng = np.random.default_rng(s)
    x = rng.standard_normal((2, 2, s, s)).astype(dtype)
    upper = np.triu(np.ones((s, s), bool), 1)
    junk = x.copy()
    junk[..., upper] = np.where(rng.random(upper.sum()) < 0.5, np.nan, np.inf).astype(dtype)
    with exact_mode():
        y = C.scaled_masked_softmax(C.to_device(junk), 0.125, True).numpy()
    sc = np.where(~upper, x * dtype(0.125), dtype(-np.inf)).astype(dtype)
    ref = O.softmax_rows(sc.reshape(-1, s)).reshape(x.shape)
    assert bits_equal(y, ref), mismatch_report(y, ref)
    y = C.scaled_masked_softmax(C.to_device(junk), 0.125, True).numpy()
    if dtype == np.float32:
        assert bits_equal(y, ref), mismatch_report(y, ref)
    else:
        assert_f64_rows_close(y, ref)


@pytest.mark.parametrize("dtype,n", [(np.float32, 10), (np.float32, 1024), (np.float64, 777)])
def test_softmax_adjoint(dtype, n):
    rng = np.random.default_rng(6)
    yv = O.softmax_rows(rng.standard_normal((256, n)).astype(dtype))
    g = rng.standard_normal((256, n)).astype(dtype)
    dx = C.softmax_adjoint(C.to_device(yv), C.to_device(g)).numpy()
    assert bits_equal(dx, O.softmax_adjoint_rows(yv, g))


@pytest.mark.parametrize("dtype,shape", [(np.float32, (4096, 1024)), (np.float32, (100, 333)),
                                         (np.float64, (512, 1024))])
def test_layer_norm_bit_exact(dtype, shape):
    rng = np.random.default_rng(7)
    x = rng.standard_normal(shape).astype(dtype)
    g = rng.standard_normal(shape[-1]).astype(dtype)
    b = rng.standard_normal(shape[-1]).astype(dtype)
    y = C.layer_norm(C.to_device(x), C.to_device(g), C.to_device(b), 1e-5).numpy()
    ref = O.layer_norm_rows(x, g, b, dtype(1e-5))
    assert bits_equal(y, ref), mismatch_report(y, ref)


def test_relu_and_adjoint_bit_rules():
    rng = np.random.default_rng(8)
    x = rng.standard_normal(1 << 20).astype(np.float32)
    x[:6] = [-0.0, 0.0, np.nan, -np.inf, np.inf, -1.0]
    x[6:8] = np.array([0x7FC01234, 0xFFC00001], np.uint32).view(np.float32)
    g = rng.standard_normal(x.size).astype(np.float32)
    assert bits_equal(C.relu(C.to_device(x)).numpy(), O.relu(x))
    assert bits_equal(C.relu_adjoint(C.to_device(x), C.to_device(g)).numpy(), O.relu_adjoint(x, g))


@pytest.mark.parametrize("n", [4, 1023, 1024 * 512 + 3])
def test_dropout_and_replay_bit_exact(n):
    key = O.fold_in(44, 7)
    x = np.random.default_rng(9).standard_normal(n).astype(np.float32)
    y = C.dropout(key, C.to_device(x), 0.1).numpy()
    assert bits_equal(y, O.dropout(key, x, np.float32(0.1)))
    g = np.random.default_rng(10).standard_normal(n).astype(np.float32)
    dx = C.dropout_replay(key, C.to_device(g), 0.1).numpy()
    assert bits_equal(dx, O.dropout_replay(key, g, np.float32(0.1)))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("rate", [0.1, 0.3, 0.7, 0.0])
def test_dropout_quotient_special_values(rate, dtype):
    """The kept quotient x / (1 - rate) at the edges of the format: binary32
    subnormals (inputs and results), values that overflow to inf once
    divided, inf, NaN (canonical on output) and signed zeros; a random bulk
    sets the rounding of ordinary quotients."""
    fi = np.finfo(dtype)
    special = np.array([fi.tiny, fi.tiny / 3, -fi.tiny / 7, fi.smallest_subnormal, fi.max, -fi.max, fi.max * 0.8,
                        np.inf, -np.inf, np.nan, 0.0, -0.0, 1.0, 3.0, -7.5], dtype)
    rng = np.random.default_rng(17)
    bulk = (rng.standard_normal(40000) * np.exp2(rng.integers(-140, 120, 40000).astype(np.float64))).astype(dtype)
    x = np.concatenate([np.tile(special, 64), bulk])
    key = 0x1234_5678_9ABC_DEF0
    with np.errstate(all="ignore"):
        y = C.dropout(key, C.to_device(x), rate).numpy()
        ref = O.dropout(key, x, dtype(rate))
    assert bits_equal(y, ref)


def test_dropout_fixed_stream_golden():
    left, right = O.split(42)
    ones = np.ones(4, np.float32)
    assert C.dropout(right, C.to_device(ones), 0.5).numpy().tolist() == [2.0, 2.0, 0.0, 0.0]
    assert C.dropout_replay(left, C.to_device(ones), 0.5).numpy().tolist() == [2.0, 0.0, 0.0, 2.0]


def test_dropout_invalid_rate_is_domain_error():
    x = C.to_device(np.ones(4, np.float32))
    with pytest.raises(C.ChelisError, match="numeric trap: domain in dropout at f32"):
        C.dropout(1, x, 1.0)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_uniform_like_bit_exact(dtype):
    out = C.empty((100003,), dtype)
    C.uniform_like(12345, -1.0, 1.0, out)
    assert bits_equal(out.numpy(), O.uniform_like(12345, dtype(-1.0), dtype(1.0), 100003, dtype))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_streamed_maps_over_whole_rounds_bit_exact(dtype):
    """Dropout, its replay and uniform_like run a resident grid that walks
    whole rounds of vectors unchecked and then one checked round: at
    3 * 2^23 + 5 elements every thread takes several whole rounds (the
    smaller sizes above take only the checked one), the checked round holds
    a partial vector count and the scalar tail one element."""
    n = 3 * (1 << 23) + 5
    key = O.fold_in(44, 9)
    x = np.random.default_rng(21).standard_normal(n).astype(dtype)
    assert bits_equal(C.dropout(key, C.to_device(x), 0.1).numpy(), O.dropout(key, x, dtype(0.1)))
    assert bits_equal(C.dropout_replay(key, C.to_device(x), 0.3).numpy(), O.dropout_replay(key, x, dtype(0.3)))
    out = C.empty((n,), dtype)
    C.uniform_like(777, -2.0, 3.0, out)
    assert bits_equal(out.numpy(), O.uniform_like(777, dtype(-2.0), dtype(3.0), n, dtype))


def gelu_f32_close(y, ref, x):
    """The binary32 default-mode GELU bar: within 1e-6 relative of the Phi
    graph (ten times inside the north star's 1e-5), with an absolute floor
    of 2^-146 for subnormal results; NaN, the infinities, the signed zeros
    and the inputs below -12.5 (the graph's own path) bit for bit."""
    y64, r64 = y.astype(np.float64), ref.astype(np.float64)
    close = np.abs(y64 - r64) <= 1e-6 * np.abs(r64) + 2.0 ** -146
    exact = np.isnan(x) | np.isinf(x) | (x == 0) | (x < -12.5)
    same = y.view(np.uint32) == ref.view(np.uint32)
    return (same | (close & ~exact)).all(), float(np.nanmax(np.abs(y64 - r64) / np.maximum(np.abs(r64), 1e-300)))


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_gelu(dtype, exact):
    rng = np.random.default_rng(12)
    x = np.concatenate([rng.standard_normal(1 << 20) * 3, np.linspace(-80, 80, 4001),
                        [np.inf, -np.inf, np.nan, 0.0, -0.0, -12.5, -12.499999, 1e-40, -1e-40, 14.0, 15.0]]).astype(dtype)
    prev = C.set_exact(exact)
    try:
        y = C.gelu(C.to_device(x)).numpy()
    finally:
        C.set_exact(prev)
    ref = O.gelu(x)
    if dtype == np.float32:
        if exact:
            # every leaf correctly rounded: the whole Phi graph matches bit for bit
            assert bits_equal(y, ref), mismatch_report(y, ref)
        else:
            ok, worst = gelu_f32_close(y, ref, x)
            assert ok, worst
        return
    both_nan = np.isnan(y) & np.isnan(ref)
    ok = both_nan | (y == ref) | (np.abs(y - ref) <= 1e-12 * np.abs(ref))
    assert ok.all(), (x[~ok][:5], y[~ok][:5], ref[~ok][:5])


@pytest.mark.parametrize("op", ["log", "erfc", "tanh"])
def test_f32_transcendental_chain_leaves_bit_exact(op):
    """The f32 log / erfc / tanh chain leaves against CORE-MATH, including
    the six inputs the device corrects through its exception table."""
    rng = np.random.default_rng(14)
    x = (rng.standard_normal(1 << 18) * 4).astype(np.float32)
    if op == "log":
        x = np.abs(x)
    special = np.array([0x3C413D3A, 0x41178FEB, 0x4C5D65A5, 0x65D890D3, 0x6F31A8EC, 0xB76C9F62, 0x7F800000,
                        0xFF800000, 0x7FC00000, 0x00000001, 0x80000000, 0x3F800000], np.uint32).view(np.float32)
    x = np.concatenate([x, special])
    out = C.empty(x.shape, np.float32)
    C.fused_elementwise(C.fused_chain([(op, 0)]), [C.to_device(x)], out)
    fn = {"log": O.lib().orc_logf, "erfc": O.lib().orc_erfcf, "tanh": O.lib().orc_tanhf}[op]
    ref = np.array([fn(v) for v in x], np.float32)
    y = out.numpy()
    assert bits_equal(y, ref), mismatch_report(y, ref)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_fused_chain_flat_paths(dtype):
    """Flat maps: 16-byte vectors with a ragged tail, a scalar broadcast
    operand, and an input one element off 16-byte alignment (scalar path)."""
    rng = np.random.default_rng(15)
    n = 4099
    a, b = rng.standard_normal(n + 1).astype(dtype), rng.standard_normal(n).astype(dtype)
    s = np.array(rng.standard_normal(), dtype)
    da, db, ds = C.to_device(a), C.to_device(b), C.to_device(s)
    ch = C.fused_chain([("mul", 0, 2), ("sub", ("s", 0), 1), ("exp", ("s", 1))])
    out = C.empty((n,), dtype)
    C.fused_elementwise(ch, [da.view((n,), (1,)), db, ds.view((n,), (0,))], out)
    fn = O.lib().orc_expf if dtype == np.float32 else O.lib().orc_exp
    exp = lambda v: np.array([fn(e) for e in v], dtype)  # noqa: E731
    t = (a[:n] * s - b).astype(dtype)
    assert bits_equal(out.numpy(), exp(t)), mismatch_report(out.numpy(), exp(t))
    out2 = C.empty((n,), dtype)
    C.fused_elementwise(ch, [da.view((n,), (1,), 1), db, ds.view((n,), (0,))], out2)
    t2 = (a[1:] * s - b).astype(dtype)
    assert bits_equal(out2.numpy(), exp(t2)), mismatch_report(out2.numpy(), exp(t2))


def test_fused_chain_sgd_and_broadcast():
    """A FusedElem chain w - lr * g plus a bias-broadcast chain relu(x + b)."""
    rng = np.random.default_rng(13)
    w = rng.standard_normal((784, 512)).astype(np.float32)
    g = rng.standard_normal((784, 512)).astype(np.float32)
    lr = np.float32(0.01)
    ch = C.fused_chain([("const", 0, 0, 0.01), ("mul", ("s", 0), 1), ("sub", 0, ("s", 1))])
    out = C.empty(w.shape, np.float32)
    C.fused_elementwise(ch, [C.to_device(w), C.to_device(g)], out)
    assert bits_equal(out.numpy(), (w - lr * g).astype(np.float32))
    x = rng.standard_normal((1024, 512)).astype(np.float32)
    b = rng.standard_normal(512).astype(np.float32)
    bd = C.to_device(b)
    bview = bd.view((1024, 512), (0, 1))
    ch2 = C.fused_chain([("add", 0, 1), ("relu", ("s", 0), 0)])
    out2 = C.empty(x.shape, np.float32)
    C.fused_elementwise(ch2, [C.to_device(x), bview], out2)
    assert bits_equal(out2.numpy(), O.relu((x + b).astype(np.float32)))


def test_fused_chain_transposed_operand_and_ops():
    rng = np.random.default_rng(14)
    a = rng.standard_normal((300, 200)).astype(np.float64)
    bt = rng.standard_normal((200, 300)).astype(np.float64)
    ad, bd = C.to_device(a), C.to_device(bt)
    bview = bd.view((300, 200), (1, 300))  # b = bt^T without a copy
    steps = [("max_elem", 0, 1), ("abs", 1, 0), ("div", ("s", 0), ("s", 1)), ("sqrt", ("s", 1), 0),
             ("add", ("s", 2), ("s", 3)), ("floor", ("s", 4), 0), ("neg", ("s", 5), 0)]
    out = C.empty(a.shape, np.float64)
    C.fused_elementwise(C.fused_chain(steps), [ad, bview], out)
    b = bt.T
    s0 = np.where(np.isnan(a) | (b <= a), a, b)
    ref = -np.floor(s0 / np.abs(b) + np.sqrt(np.abs(b)))
    assert bits_equal(out.numpy(), ref)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("n_extra_inputs", [0, 5])
def test_fused_chain_every_op_vector_and_scalar_interpreters(dtype, n_extra_inputs):
    """A chain over every arithmetic op: 3 inputs + 13 steps (16 slots, the
    vector interpreter's 64 KiB LDS budget) and 8 inputs + 16 steps (24
    slots: the scalar interpreter)."""
    rng = np.random.default_rng(21)
    n = 10003
    a = rng.uniform(0.5, 2.0, n).astype(dtype)
    b = rng.uniform(0.5, 2.0, n).astype(dtype)
    c = np.array(1.75, dtype)
    steps = [("add", 0, 1), ("mul", ("s", 0), 2), ("div", ("s", 1), 1), ("recip", ("s", 2)), ("sqrt", ("s", 3)),
             ("min_elem", ("s", 4), 0), ("ceil", ("s", 0)), ("round", ("s", 1)), ("relu_adjoint", ("s", 5), ("s", 7)),
             ("sub", ("s", 8), ("s", 6)), ("const", 0, 0, 0.25), ("mul", ("s", 9), ("s", 10)), ("neg", ("s", 11))]
    if n_extra_inputs:
        steps += [("abs", ("s", 12)), ("max_elem", ("s", 13), 3), ("floor", ("s", 14))]
    extra = [rng.uniform(-1, 1, n).astype(dtype) for _ in range(n_extra_inputs)]
    ins = [C.to_device(a), C.to_device(b), C.to_device(c).view((n,), (0,))] + [C.to_device(e) for e in extra]
    out = C.empty((n,), dtype)
    C.fused_elementwise(C.fused_chain(steps), ins, out)
    s0 = a + b
    s1 = s0 * c
    s2 = s1 / b
    s3 = dtype(1) / s2
    s4 = np.sqrt(s3)
    s5 = np.where(a < s4, a, s4)
    s6, s7 = np.ceil(s0), np.rint(s1)
    s8 = np.where(dtype(0) < s5, s7, dtype(0))
    s12 = -((s8 - s6) * dtype(0.25))
    ref = s12
    if n_extra_inputs:
        s13 = np.abs(s12)
        s14 = np.where(extra[0] > s13, extra[0], s13)
        ref = np.floor(s14)
    assert bits_equal(out.numpy(), ref.astype(dtype))


def _specials(dtype):
    if dtype == np.float32:
        bits = [0x7FC0BEEF, 0xFFC00001, 0x7F800000, 0xFF800000, 0x00000000, 0x80000000, 0x00000001, 0x80000003,
                0x3F800000, 0xBF800000, 0x7F7FFFFF, 0x3F000000, 0x40490FDB, 0xC2B00000]
        return np.array(bits, np.uint32).view(np.float32)
    bits = [0x7FF800000000BEEF, 0xFFF8000000000001, 0x7FF0000000000000, 0xFFF0000000000000, 0, 0x8000000000000000,
            1, 0x8000000000000003, 0x3FF0000000000000, 0xBFF0000000000000, 0x7FEFFFFFFFFFFFFF, 0x3FE0000000000000,
            0x400921FB54442D18, 0xC086000000000000]
    return np.array(bits, np.uint64).view(np.float64)


def _canon(v):
    v = np.array(v)
    out = v.copy()
    nan = np.isnan(v)
    out[nan] = np.array([0x7FC00000], np.uint32).view(np.float32)[0] if v.dtype == np.float32 else \
        np.array([0x7FF8000000000000], np.uint64).view(np.float64)[0]
    return out


def _ref_step(op, a, b, imm, dtype):
    """One FusedElem step as the C lane evaluates it (crates/chelis-backend-c/
    src/emit.rs:6744-6895, NaN finalization per fp_env.rs:214-241): every op
    stores the canonical NaN except max_elem / min_elem, which keep the
    selected operand's bits; relu / relu_adjoint select stored bits
    ([05-OP-43]); transcendental leaves are the oracle's CORE-MATH values."""
    L = O.lib()
    leaf = {"exp": (L.orc_expf, L.orc_exp), "log": (L.orc_logf, L.orc_log), "tanh": (L.orc_tanhf, L.orc_tanh),
            "erfc": (L.orc_erfcf, L.orc_erfc)}
    with np.errstate(all="ignore"):
        if op in leaf:
            fn = leaf[op][0 if dtype == np.float32 else 1]
            return np.array([fn(v) for v in a], dtype)
        if op == "max_elem":
            return np.where(np.isnan(a) | (~np.isnan(b) & (a >= b)), a, b)
        if op == "min_elem":
            return np.where(np.isnan(a) | (~np.isnan(b) & (a <= b)), a, b)
        if op == "relu":
            return np.where(a < 0, dtype(0), a)
        if op == "relu_adjoint":
            return np.where(dtype(0) < a, b, dtype(0))
        if op == "const":
            return np.full(a.shape, dtype(imm))
        f = {"add": lambda: a + b, "sub": lambda: a - b, "mul": lambda: a * b, "div": lambda: a / b,
             "neg": lambda: -a, "recip": lambda: dtype(1) / a, "sqrt": lambda: np.sqrt(a), "abs": lambda: np.abs(a),
             "floor": lambda: np.floor(a), "ceil": lambda: np.ceil(a), "round": lambda: np.rint(a)}[op]
        return _canon(f().astype(dtype))


SPECIAL_CHAINS = [
    [("add", 0, 1), ("sub", 0, 1), ("mul", 0, 1), ("div", 0, 1), ("max_elem", 0, 1), ("min_elem", 1, 0),
     ("neg", 0), ("recip", 1), ("sqrt", 0), ("abs", 1), ("floor", 0), ("ceil", 1), ("round", 0),
     ("relu", 1), ("relu_adjoint", 0, 1), ("max_elem", ("s", 4), ("s", 14))],
    [("exp", 0), ("log", 1), ("tanh", 0), ("erfc", 1), ("min_elem", ("s", 0), ("s", 1)),
     ("max_elem", ("s", 2), ("s", 3)), ("const", 0, 0, -0.0), ("add", ("s", 6), ("s", 4)),
     ("mul", ("s", 7), ("s", 5)), ("relu", ("s", 8))],
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("chain_id", [0, 1])
@pytest.mark.parametrize("last_step", list(range(16)))
@pytest.mark.parametrize("n_inputs", [2, 8])
def test_fused_chain_special_values_both_interpreters(dtype, chain_id, last_step, n_inputs):
    """NaN payloads (quiet, negative), +-inf, +-0, subnormals, the largest
    finite value and ordinary values, every ordered pair of them, through
    every step kind, with a ragged tail (n % (16 / itemsize) != 0). Two
    inputs take the 16-byte vector interpreter; eight inputs (six unused)
    take the one-element LDS-slot interpreter. Each chain is cut after every
    step in turn, so each step's result is observed directly."""
    steps = SPECIAL_CHAINS[chain_id]
    if last_step >= len(steps):
        pytest.skip("chain shorter than the cut")
    steps = steps[:last_step + 1]
    sp = _specials(dtype)
    a = np.repeat(sp, sp.size)
    b = np.tile(sp, sp.size)
    rng = np.random.default_rng(31)
    pad = 7
    a = np.concatenate([a, (rng.standard_normal(pad) * 3).astype(dtype)])
    b = np.concatenate([b, (rng.standard_normal(pad) * 3).astype(dtype)])
    n = a.size
    ins = [C.to_device(a), C.to_device(b)] + [C.to_device(np.zeros(n, dtype)) for _ in range(n_inputs - 2)]
    out = C.empty((n,), dtype)
    C.fused_elementwise(C.fused_chain(steps), ins, out)
    vals = []
    for st in steps:
        op = st[0]
        args = [st[1] if len(st) > 1 else 0, st[2] if len(st) > 2 else 0]
        av = [vals[x[1]] if isinstance(x, tuple) else (a, b)[x] if x < 2 else np.zeros(n, dtype) for x in args]
        vals.append(_ref_step(op, av[0], av[1], st[3] if len(st) > 3 else 0.0, dtype))
    ref = vals[-1].astype(dtype)
    y = out.numpy()
    if dtype == np.float64 and any(st[0] in ("log", "tanh", "erfc") for st in steps):
        # binary64 log / tanh / erfc leaves are the device library's (within
        # 1 ulp, the 1e-12 relative contract); specials keep exact bits
        finite = np.isfinite(ref) & (ref != 0)
        assert bits_equal(y[~finite], ref[~finite]), mismatch_report(y[~finite], ref[~finite])
        assert np.all(np.abs(y[finite] - ref[finite]) <= 1e-12 * np.abs(ref[finite]))
    else:
        assert bits_equal(y, ref), mismatch_report(y, ref)


def _attention_ref(q, k, v, scale):
    """float64 reference of softmax(where(j <= i, q.k^T * scale, -inf)).v."""
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), k.astype(np.float64)) * scale
    n = s.shape[-1]
    s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", p, v.astype(np.float64))


@pytest.mark.parametrize("B,H,S", [(1, 1, 64), (2, 3, 192), (2, 16, 512)])
def test_causal_attention_fused(B, H, S):
    """The fused attention kernel against a float64 reference of the graph,
    within the binary32 tolerance (normwise 1e-5)."""
    rng = np.random.default_rng(B * 100 + H * 10 + S)
    q, k, v = (rng.standard_normal((B, H, S, 64)).astype(np.float32) for _ in range(3))
    o = C.causal_attention(C.to_device(q), C.to_device(k), C.to_device(v), 0.125).numpy()
    ref = _attention_ref(q, k, v, 0.125)
    assert np.abs(o - ref).max() <= 1e-5 * np.abs(ref).max()


def test_causal_attention_head_interleaved_views():
    """q, k, v and o as [B, H, S, 64] views of [B, S, H*64] storage (the
    transformer block's projections), large logits (scale 1) so the running
    maxima move."""
    B, S, H = 2, 256, 4
    rng = np.random.default_rng(9)
    raw = [rng.standard_normal((B, S, H * 64)).astype(np.float32) * 2 for _ in range(3)]
    dev = [C.to_device(x) for x in raw]
    views = [d.view((B, H, S, 64), (S * H * 64, 64, H * 64, 1)) for d in dev]
    out = C.empty((B, S, H * 64), np.float32)
    ov = out.view((B, H, S, 64), (S * H * 64, 64, H * 64, 1))
    C.causal_attention(views[0], views[1], views[2], 1.0, ov)
    q, k, v = (x.reshape(B, S, H, 64).transpose(0, 2, 1, 3) for x in raw)
    ref = _attention_ref(q, k, v, 1.0).transpose(0, 2, 1, 3).reshape(B, S, H * 64)
    o = out.numpy()
    assert np.abs(o - ref).max() <= 1e-5 * np.abs(ref).max()


def test_causal_attention_rejects_unsupported_shapes():
    q = C.to_device(np.zeros((1, 1, 96, 64), np.float32))
    with pytest.raises(C.ChelisError):
        C.causal_attention(q, q, q, 0.125, C.empty((1, 1, 96, 64), np.float32))


LONG_ROWS = [(np.float32, 3, 65537), (np.float32, 2, 200_003), (np.float64, 3, 32769), (np.float64, 2, 100_001)]


@pytest.mark.parametrize("dtype,rows,n", LONG_ROWS)
def test_long_rows_bit_exact(dtype, rows, n):
    """Rows past the register capacity (65 536 f32 / 32 768 f64 values) run
    as reductions and chains in the row kernels' primitive order: softmax,
    its adjoint and layer norm stay bit-exact against the oracle; strided
    rows included."""
    rng = np.random.default_rng(n + rows)
    x = (rng.standard_normal((rows, n)) * 3).astype(dtype)
    g = rng.standard_normal((rows, n)).astype(dtype)
    gamma = (1 + 0.1 * rng.standard_normal(n)).astype(dtype)
    beta = (0.1 * rng.standard_normal(n)).astype(dtype)
    # x as a strided view: rows padded by 5 elements
    buf = np.zeros((rows, n + 5), dtype)
    buf[:, :n] = x
    dbuf = C.to_device(buf)
    xv = dbuf.view((rows, n), (n + 5, 1))
    y = C.softmax(xv).numpy()
    ref = O.softmax_rows(x)
    assert bits_equal(y, ref)
    dx = C.softmax_adjoint(C.to_device(ref), C.to_device(g)).numpy()
    assert bits_equal(dx, O.softmax_adjoint_rows(ref, g))
    ln = C.layer_norm(xv, C.to_device(gamma), C.to_device(beta), 1e-5).numpy()
    assert bits_equal(ln, O.layer_norm_rows(x, gamma, beta, 1e-5))


def _attention_oracle(q, k, v, scale):
    """The C oracle's composition of spec/05 section 4.7's graph per (batch,
    head): canonical-tree q.k^T, the scale at binary32, where(j <= i, s,
    -inf), the oracle's softmax rows, canonical-tree P.v."""
    B, H, S, _ = q.shape
    out = np.empty(q.shape, np.float32)
    mask = np.tril(np.ones((S, S), bool))
    for b in range(B):
        for h in range(H):
            s = O.matmul(q[b, h], np.ascontiguousarray(k[b, h].T)) * np.float32(scale)
            p = O.softmax_rows(np.where(mask, s, np.float32(-np.inf)).astype(np.float32))
            out[b, h] = O.matmul(p, v[b, h])
    return out


@pytest.mark.parametrize("B,H,S", [(2, 3, 192), (1, 2, 512)])
def test_causal_attention_fused_against_the_oracle(B, H, S):
    """The fused attention (MFMA products, online softmax) against the C
    oracle's composition of the same graph: normwise 1e-5 and, where the
    output is not small against its rms, 1e-5 relative per element (the
    binary32 bar of the north star)."""
    rng = np.random.default_rng(B * 1000 + H * 10 + S)
    q, k, v = (rng.standard_normal((B, H, S, 64)).astype(np.float32) for _ in range(3))
    o = C.causal_attention(C.to_device(q), C.to_device(k), C.to_device(v), 0.125).numpy().astype(np.float64)
    ref = _attention_oracle(q, k, v, 0.125).astype(np.float64)
    assert np.abs(o - ref).max() <= 1e-5 * np.abs(ref).max()
    big = np.abs(ref) >= np.sqrt(np.mean(ref ** 2))
    assert np.all(np.abs(o - ref)[big] <= 1e-5 * np.abs(ref)[big])

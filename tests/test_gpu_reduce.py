"""GPU parity of the axis reductions (chelis_hip_reduce, chelis_hip_count)
against the C oracle: sums are the canonical tree ([05-OP-30]) bit for bit,
max/min keep the first NaN and the first stored representation ([05-OP-12]),
argmax/argmin the first index, counts are exact with the reference kernel's
error code 1 for a byte that is not 0 or 1
(crates/chelis-backend-hip/src/kernels.rs:375-557)."""
import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def setup_module(_m):
    O.build()


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


SHAPES = [((1,), 0), ((7,), 0), ((64, 1000), 1), ((64, 1000), 0), ((3, 257, 5), 1), ((1024, 10), 1),
          ((1024, 512), 0), ((2, 3, 4097), 2), ((4100, 3), 0), ((33, 65537), 1)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape,axis", SHAPES)
def test_sum_and_max_bit_exact(shape, axis, dtype):
    rng = np.random.default_rng(sum(shape) + axis)
    x = (rng.standard_normal(shape) * 3).astype(dtype)
    d = C.to_device(x)
    assert bits_equal(C.reduce("sum", d, axis).numpy(), O.sum_axis(x, axis))
    assert bits_equal(C.reduce("max", d, axis).numpy(), O.max_axis(x, axis))
    assert bits_equal(C.reduce("min", d, axis).numpy(), -O.max_axis(-x, axis))
    am = C.reduce("argmax", d, axis).numpy()
    assert np.array_equal(am, np.argmax(x, axis))


def test_max_first_nan_and_signed_zero():
    x = np.array([[0.0, -0.0, 1.0, np.nan, 2.0], [-0.0, 0.0, -0.0, 0.0, -1.0], [1.0, 3.0, 3.0, -np.inf, 0.0]],
                 np.float32)
    x[0, 3] = np.array([0x7FC0BEEF], np.uint32).view(np.float32)[0]  # NaN with a payload
    d = C.to_device(x)
    mx = C.reduce("max", d, 1).numpy()
    assert bits_equal(mx, O.max_axis(x, 1))
    assert np.array_equal(C.reduce("argmax", d, 1).numpy(), [3, 0, 1])


def test_sum_of_fused_chain_leaf():
    """reduce_fused: sum over the axis of (x - m) * (x - m) with m broadcast."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((512, 1024)).astype(np.float32)
    m = x.mean(1, dtype=np.float32)
    dx, dm = C.to_device(x), C.to_device(m)
    mv = dm.view((512, 1024), (1, 0))
    ch = C.fused_chain([("sub", 0, 1), ("mul", ("s", 0), ("s", 0))])
    out = C.reduce("sum", [dx, mv], 1, chain=ch).numpy()
    leaf = ((x - m[:, None]) * (x - m[:, None])).astype(np.float32)
    assert bits_equal(out, O.sum_axis(leaf, 1))


def test_empty_axis():
    d = C.empty((4, 0), np.float64)
    assert bits_equal(C.reduce("sum", d, 1).numpy(), np.zeros(4))
    with pytest.raises(C.ChelisError, match="numeric trap: domain in max_reduce at f64"):
        C.reduce("max", d, 1)


@pytest.mark.parametrize("shape,axis", [((1024, 512), 1), ((1024, 512), 0), ((7, 100003), 1)])
def test_count_exact(shape, axis):
    x = (np.random.default_rng(6).random(shape) < 0.3).astype(np.uint8)
    out, err = C.count(C.to_device(x), axis)
    ref, rerr = O.count_axis(x, axis)
    assert err == 0 == rerr and np.array_equal(out.numpy(), ref)


def test_count_rejects_non_bool_byte():
    x = np.zeros((4, 64), np.uint8)
    x[2, 17] = 2
    out, err = C.count(C.to_device(x), 1)
    assert err == 1 and O.count_axis(x, 1)[1] == 1


# Contiguous rows take the 16-byte path (reduce_rows_vec_kernel): row starts
# aligned to 16 bytes, leaves at stride 1. The views below keep the rows
# aligned while the row length leaves a partial vector at the end, and the
# long rows take several passes (the later argmax passes use the scalar
# kernel, which carries the partial indices).
VEC_CASES = [((64, 1024), 1001), ((5, 8), 7), ((40, 4104), 4100), ((3, 300000), 300000), ((2, 70000), 69999)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("alloc,n", VEC_CASES)
def test_contiguous_rows_partial_vector_and_passes(alloc, n, dtype):
    rng = np.random.default_rng(alloc[1] + n)
    buf = (rng.standard_normal(alloc) * 3).astype(dtype)
    x = np.ascontiguousarray(buf[:, :n])
    d = C.to_device(buf).view((alloc[0], n), (alloc[1], 1))
    assert bits_equal(C.reduce("sum", d, 1).numpy(), O.sum_axis(x, 1))
    assert bits_equal(C.reduce("max", d, 1).numpy(), O.max_axis(x, 1))
    assert bits_equal(C.reduce("min", d, 1).numpy(), -O.max_axis(-x, 1))
    assert np.array_equal(C.reduce("argmax", d, 1).numpy(), np.argmax(x, 1))
    assert np.array_equal(C.reduce("argmin", d, 1).numpy(), np.argmin(x, 1))


def test_contiguous_rows_nan_and_ties_in_vectors():
    """First NaN / first index inside one lane's vector and across lanes."""
    x = np.zeros((4, 1024), np.float32)
    x[0, [5, 6, 700]] = [np.nan, 3.0, np.nan]
    x[0, 5] = np.array([0x7FC0BEEF], np.uint32).view(np.float32)[0]
    x[1, [2, 3, 900]] = 7.0
    x[2, :] = -0.0
    x[2, 513] = 0.0
    x[3, 1023] = -np.inf
    d = C.to_device(x)
    assert bits_equal(C.reduce("max", d, 1).numpy(), O.max_axis(x, 1))
    assert bits_equal(C.reduce("min", d, 1).numpy(), -O.max_axis(-x, 1))
    assert np.array_equal(C.reduce("argmax", d, 1).numpy()[1:], np.argmax(x, 1)[1:])
    assert C.reduce("argmax", d, 1).numpy()[0] == 5


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("alloc,n", [((256, 1000), 1000), ((64, 1024), 1001), ((4, 20000), 20000)])
def test_sum_of_contiguous_chain_leaf(alloc, n, dtype):
    """reduce_fused with every input contiguous: sum((x - g) * (x - g))."""
    rng = np.random.default_rng(n)
    xb = rng.standard_normal(alloc).astype(dtype)
    gb = rng.standard_normal(alloc).astype(dtype)
    x, g = xb[:, :n], gb[:, :n]
    dx = C.to_device(xb).view((alloc[0], n), (alloc[1], 1))
    dg = C.to_device(gb).view((alloc[0], n), (alloc[1], 1))
    ch = C.fused_chain([("sub", 0, 1), ("mul", ("s", 0), ("s", 0))])
    leaf = ((x - g) * (x - g)).astype(dtype)
    assert bits_equal(C.reduce("sum", [dx, dg], 1, chain=ch).numpy(), O.sum_axis(np.ascontiguousarray(leaf), 1))
    ch2 = C.fused_chain([("sub", 0, 1), ("exp", ("s", 0), 0)])
    leaf2 = O.unary("exp", np.ascontiguousarray((x - g).astype(dtype)))
    assert bits_equal(C.reduce("max", [dx, dg], 1, chain=ch2).numpy(), O.max_axis(leaf2, 1))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape,axis", [((3, 1000, 256), 1), ((20000, 512), 0), ((130, 4100), 0), ((64, 1030), 0),
                                        ((16384, 64), 0)])
def test_column_reductions_with_special_values(shape, axis, dtype):
    """Column reductions (inner >= 64: four waves per 128-leaf group, one or
    more partial passes, widths that are and are not multiples of four):
    sum, max and min bit-identical to the oracle, with NaN, signed zeros and
    infinities placed in some columns."""
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(dtype)
    flat = x.reshape(-1, shape[-1])
    flat[5::97, 7] = np.nan
    flat[:, 9] = -0.0
    flat[3::11, 9] = 0.0
    flat[:, 11] = 0.0
    flat[::13, 13] = -np.inf
    d = C.to_device(x)
    assert bits_equal(C.reduce("sum", d, axis).numpy(), O.sum_axis(x, axis))
    assert bits_equal(C.reduce("max", d, axis).numpy(), O.max_axis(x, axis))
    assert bits_equal(C.reduce("min", d, axis).numpy(), -O.max_axis(-x, axis))


CHAINS_BY_INPUTS = {
    1: ([("mul", 0, 0)], lambda a: a[0] * a[0]),
    3: ([("sub", 0, 1), ("mul", ("s", 0), 2)], lambda a: (a[0] - a[1]) * a[2]),
    4: ([("sub", 0, 1), ("sub", 2, 3), ("mul", ("s", 0), ("s", 1))], lambda a: (a[0] - a[1]) * (a[2] - a[3])),
}


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("n_in", [1, 3, 4])
@pytest.mark.parametrize("rows,n", [(2048, 4096), (256, 8000), (512, 2000), (513, 2000), (300, 1000), (64, 1001),
                                    (8, 2500)])
def test_contiguous_chain_leaf_by_input_count(n_in, rows, n, dtype):
    """Chain leaves over 1, 3 and 4 contiguous inputs at row counts and
    lengths that put 1, 2 or 4 segments on a wave (ragged tails included),
    with the row's 2 or 4 groups joined inside the workgroup ([2048,4096]
    and [512,2000] f32, [512,2000] f64) or by further passes ([513,2000]:
    the rows do not fill whole workgroups; [256,8000]: more than four
    groups): sum and max bit-identical to the oracle's tree over the same
    leaves, the max with NaN leaves in some rows."""
    rng = np.random.default_rng(rows * 7 + n_in)
    width = (n + 3) // 4 * 4
    bufs = [rng.standard_normal((rows, width)).astype(dtype) for _ in range(n_in)]
    bufs[0][1::5, n // 3] = np.nan
    arrs = [b[:, :n] for b in bufs]
    devs = [C.to_device(b).view((rows, n), (width, 1)) for b in bufs]
    steps, ref = CHAINS_BY_INPUTS[n_in]
    ch = C.fused_chain(steps)
    leaf = np.ascontiguousarray(ref(arrs).astype(dtype))
    assert bits_equal(C.reduce("sum", devs, 1, chain=ch).numpy(), O.sum_axis(leaf, 1))
    assert bits_equal(C.reduce("max", devs, 1, chain=ch).numpy(), O.max_axis(leaf, 1))


@pytest.mark.parametrize("alloc,n", [((6, 4112), 4112), ((6, 4112), 4100), ((3, 16), 5)])
def test_count_contiguous_rows(alloc, n):
    buf = (np.random.default_rng(n).random(alloc) < 0.6).astype(np.uint8)
    x = np.ascontiguousarray(buf[:, :n])
    out, err = C.count(C.to_device(buf).view((alloc[0], n), (alloc[1], 1)), 1)
    ref, rerr = O.count_axis(x, 1)
    assert err == 0 == rerr and np.array_equal(out.numpy(), ref)


@pytest.mark.parametrize("col", [17, 4099])
def test_count_contiguous_rows_rejects_non_bool_byte(col):
    """A byte other than 0/1 in the 16-byte body (col 17) or the scalar tail."""
    buf = np.ones((4, 4112), np.uint8)
    buf[2, col] = 0x81
    x = np.ascontiguousarray(buf[:, :4100])
    out, err = C.count(C.to_device(buf).view((4, 4100), (4112, 1)), 1)
    assert err == 1 and O.count_axis(x, 1)[1] == 1


# Columns with at least 64 of them take reduce_cols4_kernel: 128-leaf groups
# per block (four 32-leaf wave groups joined in order). Column counts that
# leave a partial 64-column block, several passes, indices carried through
# the passes.
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape,axis", [((20000, 100), 0), ((3, 300, 70), 1), ((129, 64), 0), ((5, 4096), 0)])
def test_column_blocks_bit_exact(shape, axis, dtype):
    rng = np.random.default_rng(sum(shape))
    x = (rng.standard_normal(shape) * 3).astype(dtype)
    x.flat[::97] = x.flat[1::97]  # repeated values: first-index ties
    d = C.to_device(x)
    assert bits_equal(C.reduce("sum", d, axis).numpy(), O.sum_axis(x, axis))
    assert bits_equal(C.reduce("max", d, axis).numpy(), O.max_axis(x, axis))
    assert bits_equal(C.reduce("min", d, axis).numpy(), -O.max_axis(-x, axis))
    assert np.array_equal(C.reduce("argmax", d, axis).numpy(), np.argmax(x, axis))
    assert np.array_equal(C.reduce("argmin", d, axis).numpy(), np.argmin(x, axis))


def test_column_blocks_chain_leaf():
    rng = np.random.default_rng(31)
    x = rng.standard_normal((1000, 96)).astype(np.float32)
    g = rng.standard_normal((1000, 96)).astype(np.float32)
    ch = C.fused_chain([("sub", 0, 1), ("mul", ("s", 0), ("s", 0))])
    out = C.reduce("sum", [C.to_device(x), C.to_device(g)], 0, chain=ch).numpy()
    assert bits_equal(out, O.sum_axis(((x - g) * (x - g)).astype(np.float32), 0))


PROD_SHAPES = [((1,), 0), ((7,), 0), ((64, 1000), 1), ((64, 1000), 0), ((3, 257, 5), 1), ((2, 3, 4097), 2),
               ((4100, 3), 0), ((5, 0), 1)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape,axis", PROD_SHAPES)
def test_prod_is_the_left_fold_bit_exact(shape, axis, dtype):
    """ProdReduce: the C lane's left fold from 1 (oracle prod_axis), with
    values near 1 so long folds stay finite, plus planted zeros, infinities,
    NaN payloads and subnormals whose order decides the result."""
    rng = np.random.default_rng(sum(shape) + 3 * axis)
    x = rng.uniform(0.97, 1.03, shape).astype(dtype)
    flat = x.reshape(-1)
    if flat.size > 40:
        tiny = np.finfo(dtype).smallest_subnormal
        big = np.finfo(dtype).max
        flat[[3, 11, 17, 29, 31]] = [0.0, np.inf, tiny, big, -0.0]
        flat[37] = np.array([0x7FC0BEEF], np.uint32).view(np.float32)[0] if dtype == np.float32 else \
            np.array([0x7FF800000000BEEF], np.uint64).view(np.float64)[0]
    d = C.to_device(x)
    got = C.reduce("prod", d, axis).numpy()
    assert bits_equal(got, O.prod_axis(x, axis))


def test_prod_refuses_a_chain_leaf():
    x = C.to_device(np.ones((4, 8), np.float32))
    ch = C.fused_chain([("mul", 0, 0)])
    with pytest.raises(C.ChelisError, match="status 2"):
        C.reduce("prod", [x], 1, chain=ch)


def test_count_deferred_trap_channel():
    """Deferred counts do not wait: their codes accumulate in the device's
    trap channel until chelis_hip_trap_status reads and clears it."""
    rng = np.random.default_rng(12)
    good = (rng.random((256, 1000)) < 0.5).astype(np.uint8)
    bad = good.copy()
    bad[100, 999] = 7
    assert C.trap_status() == 0
    out, err = C.count(C.to_device(good), 1, deferred=True)
    assert err is None and C.trap_status() == 0
    assert np.array_equal(out.numpy(), good.sum(1))
    C.count(C.to_device(bad), 1, deferred=True)
    C.count(C.to_device(good), 1, deferred=True)
    assert C.trap_status() == 1
    assert C.trap_status() == 0
    # a synchronous count neither reads nor clears the channel
    C.count(C.to_device(bad), 0, deferred=True)
    _, e = C.count(C.to_device(good), 1)
    assert e == 0 and C.trap_status() == 1


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape,axis", [((16384, 4096), 0), ((128, 4), 0), ((256, 1026), 0), ((3, 1024, 520), 1),
                                        ((32768, 1000), 0), ((384, 4100), 0), ((1280, 300), 0),
                                        ((32896, 64), 0), ((2, 128, 8), 1)])
def test_column_sums_at_many_shapes(shape, axis, dtype):
    """Column sums whose leaf counts are and are not multiples of the
    128-leaf groups, whose partial counts are and are not powers of two, and
    whose column counts are narrower and wider than a workgroup's 64 columns:
    the canonical tree bit for bit, with NaN, signed zeros and infinities in
    some columns, twice in a row."""
    rng = np.random.default_rng(sum(shape) + 3)
    x = rng.standard_normal(shape).astype(dtype)
    flat = np.moveaxis(x, axis, 0).reshape(shape[axis], -1)
    flat[5::97, 1] = np.nan
    flat[:, 2] = -0.0
    flat[3::11, 2] = 0.0
    flat[::13, 3] = -np.inf
    d = C.to_device(x)
    ref = O.sum_axis(x, axis)
    for _ in range(2):
        assert bits_equal(C.reduce("sum", d, axis).numpy(), ref)


def test_column_sum_of_a_strided_view():
    """A column sum over rows whose stride is not a whole number of 16-byte
    vectors: the same values, the same bits as over the dense copy."""
    rng = np.random.default_rng(77)
    big = rng.standard_normal((1024, 1031)).astype(np.float32)
    d = C.to_device(big)
    view = d.view((1024, 1024), (1031, 1))
    assert bits_equal(C.reduce("sum", view, 0).numpy(), O.sum_axis(np.ascontiguousarray(big[:, :1024]), 0))

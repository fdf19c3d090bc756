"""chelis_hip_reduce_static, the allocation-free reduce entry: its results
against chelis_hip_reduce's (the entry it mirrors) bit for bit, on two calls
in a row with the second input smaller, through the C ABI; no scratch
request and no device allocation across its calls
(chelis_hip_allocation_counts, which does see the allocating entry's); and
the clear refusal of a reduction whose partials exceed the fixed array."""
import numpy as np
import pytest

import chelis_amd as C

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


CASES = [
    # (op, dtype, first shape, second (smaller) shape, axis): multi-pass
    # rows, multi-pass columns (four-wave groups and 32-leaf groups), argmax
    # partials with indices, one-pass rows
    ("sum", np.float32, (64, 1 << 20), (48, 300000), 1),
    ("max", np.float64, (8, 1 << 19), (3, 70001), 1),
    ("sum", np.float32, (16384, 4096), (9000, 1000), 0),
    ("argmax", np.float32, (16384, 4096), (5000, 3000), 0),
    ("min", np.float64, (1 << 16, 24), (20000, 7), 0),
    ("argmin", np.float64, (33, 1 << 18), (5, 1000), 1),
    ("sum", np.float64, (4096, 1024), (100, 1024), 1),
]


@pytest.mark.parametrize("op,dtype,shape1,shape2,axis", CASES)
def test_static_reduce_matches_the_allocating_entry(op, dtype, shape1, shape2, axis):
    rng = np.random.default_rng(sum(shape1) + axis)
    for shape in (shape1, shape2):
        x = rng.standard_normal(shape).astype(dtype)
        if op in ("argmax", "argmin"):
            x = np.round(x * 4) / 4  # ties, so the first-index rule is exercised
        d = C.to_device(x)
        ref = C.reduce(op, d, axis).numpy()
        out = C.empty(ref.shape, ref.dtype)
        C.synchronize()
        before = C.allocation_counts()
        got = C.reduce(op, d, axis, out=out, static=True)
        C.synchronize()
        # the entry's defining property: no scratch request, no allocation
        assert C.allocation_counts() == before, (op, shape)
        assert np.array_equal(bits(got.numpy()), bits(ref)), (op, shape)


def test_static_reduce_chain_leaf_twice():
    rng = np.random.default_rng(7)
    ch = C.fused_chain([("sub", 0, 1), ("mul", ("s", 0), ("s", 0))])
    for rows, n in ((512, 1 << 16), (100, 5000)):
        x = rng.standard_normal((rows, n)).astype(np.float32)
        m = rng.standard_normal(rows).astype(np.float32)
        dx, dm = C.to_device(x), C.to_device(m)
        mv = dm.view((rows, n), (1, 0))
        ref = C.reduce("sum", [dx, mv], 1, chain=ch).numpy()
        out = C.empty(ref.shape, ref.dtype)
        C.synchronize()
        before = C.allocation_counts()
        got = C.reduce("sum", [dx, mv], 1, chain=ch, out=out, static=True)
        C.synchronize()
        assert C.allocation_counts() == before
        assert np.array_equal(bits(got.numpy()), bits(ref))


def test_the_counters_see_the_allocating_entry():
    """A two-pass reduction through chelis_hip_reduce asks for scratch (a
    cached block or a new one), so the counters the static test relies on
    do move when an entry allocates."""
    d = C.to_device(np.ones((64, 1 << 20), np.float32))
    out = C.empty((64,), np.float32)
    C.synchronize()
    before = C.allocation_counts()
    C.reduce("sum", d, 1, out=out)
    C.synchronize()
    assert C.allocation_counts()[0] > before[0]


def test_static_reduce_refuses_partials_beyond_the_array():
    """32 columns of 2^21 f32 leaves: 2^16 partial groups per column in the
    first pass, 8 MiB of partials plus a second pass, over the fixed array.
    The refusal comes before anything is enqueued."""
    x = C.empty((1 << 21, 32), np.float32)
    out = C.empty((32,), np.float32)
    with pytest.raises(C.ChelisError, match="static scratch holds 8388608"):
        C.reduce("sum", x, 0, out, static=True)
    # the allocating entry takes the same request
    C.reduce("sum", x, 0, out)
    assert np.array_equal(out.numpy(), np.zeros(32, np.float32))

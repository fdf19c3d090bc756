"""GPU parity of the bfloat16 / binary16 paths against the CPU oracle.

The reference admits 16-bit tensors on HIP for sub, max_elem and min_elem
chains, relu and its adjoint, and BlasMatmul through hipblasGemmEx with a
binary32 accumulator (crates/chelis-backend-hip/src/emit.rs:2292-2319,
kernels.rs:1196-1260, runtime/chelis_hip_runtime.h:92-170). Bar:
- chains, relu, relu adjoint: bit-exact (binary32 arithmetic, one rounding
  to 16 bits per step, selections keep stored bits);
- matmul on the MFMA tiles: within one 16-bit rounding of the float64
  product plus the binary32 accumulation bound K * 2^-24 * sum |a b|
  (the reference's own test allows 1e-2 relative for bf16, 1e-3 for f16,
  crates/chelis-backend-hip/tests/bf16_f16_matmul.rs:693-784);
- matmul with CHELIS_MATMUL_EXACT: bit-exact with the oracle's decode,
  binary32 canonical tree, encode.
bf16 tensors are carried as np.uint16 bit patterns, f16 as np.float16.
"""
import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
KINDS = ["bf16", "f16"]
SPECIAL = {"bf16": [0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0x7FC1, 0xFFC3, 0x0001, 0x8001, 0x7F7F, 0xFF7F, 0x3F80],
           "f16": [0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0x7E01, 0xFE03, 0x0001, 0x8001, 0x7BFF, 0xFBFF, 0x3C00]}


def setup_module(_m):
    O.build()


def carrier(kind, bits):
    """Host array of the device dtype for 16-bit patterns."""
    bits = np.ascontiguousarray(bits, np.uint16)
    return bits if kind == "bf16" else bits.view(np.float16)


def bits_of(a):
    return np.ascontiguousarray(a).view(np.uint16)


def random_bits(kind, shape, seed, scale=4.0):
    rng = np.random.default_rng(seed)
    b = O.narrow_encode(kind, (rng.standard_normal(shape) * scale).astype(np.float32))
    flat = b.reshape(-1)
    sp = np.array(SPECIAL[kind], np.uint16)
    flat[: min(len(sp), flat.size)] = sp[: flat.size]
    return b


@pytest.mark.parametrize("kind", KINDS)
def test_narrow_chain_bit_exact(kind):
    n = 70001
    a, b, c = (random_bits(kind, n, s) for s in (1, 2, 3))
    ch = C.fused_chain([("sub", 0, 1), ("max_elem", ("s", 0), 2), ("min_elem", ("s", 1), 0), ("sub", ("s", 2), 1)])
    out = C.empty((n,), carrier(kind, a).dtype)
    C.fused_elementwise(ch, [C.to_device(carrier(kind, x)) for x in (a, b, c)], out)
    s0 = O.narrow_binary("sub", kind, a, b)
    s1 = O.narrow_binary("max", kind, s0, c)
    s2 = O.narrow_binary("min", kind, s1, a)
    want = O.narrow_binary("sub", kind, s2, b)
    got = bits_of(out.numpy())
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:8]


@pytest.mark.parametrize("kind", KINDS)
def test_narrow_chain_broadcast_and_strided(kind):
    """A row-broadcast operand (stride 0) and a transposed view."""
    a = random_bits(kind, (64, 96), 4)
    row = random_bits(kind, (1, 96), 5)
    big = random_bits(kind, (96, 64), 6)
    da, dr, dbig = C.to_device(carrier(kind, a)), C.to_device(carrier(kind, row)), C.to_device(carrier(kind, big))
    out = C.empty((64, 96), carrier(kind, a).dtype)
    ch = C.fused_chain([("sub", 0, 1), ("max_elem", ("s", 0), 2)])
    C.fused_elementwise(ch, [da, dr.view((64, 96), (0, 1)), dbig.view((64, 96), (1, 64))], out)
    s0 = O.narrow_binary("sub", kind, a, np.broadcast_to(row, (64, 96)))
    want = O.narrow_binary("max", kind, s0, big.T)
    assert np.array_equal(bits_of(out.numpy()), want)


@pytest.mark.parametrize("kind", KINDS)
def test_narrow_chain_rejects_other_steps(kind):
    x = C.to_device(carrier(kind, random_bits(kind, 16, 7)))
    out = C.empty((16,), x.dtype)
    with pytest.raises(C.ChelisError, match="outside sub/max_elem/min_elem"):
        C.fused_elementwise(C.fused_chain([("exp", 0)]), [x], out)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n", [8, 13, 4096 + 5])
def test_narrow_relu_and_adjoint_bit_exact(kind, n):
    x, g = random_bits(kind, n, 8 + n), random_bits(kind, n, 9 + n)
    dx, dg = C.to_device(carrier(kind, x)), C.to_device(carrier(kind, g))
    assert np.array_equal(bits_of(C.relu(dx).numpy()), O.narrow_relu(kind, x))
    assert np.array_equal(bits_of(C.relu_adjoint(dx, dg).numpy()), O.narrow_relu_adjoint(kind, x, g))


def finite_bits(kind, shape, seed):
    """Random 16-bit operands of moderate magnitude (|x| < 8, subnormals of
    the special set kept) so that binary32 sums cannot overflow."""
    b = random_bits(kind, shape, seed, 1.0)
    v = O.narrow_decode(kind, b)
    return O.narrow_encode(kind, np.clip(np.nan_to_num(v, nan=0.5, posinf=1, neginf=-1), -8, 8))


def _mm_bound(kind, a_bits, b_bits):
    a = O.narrow_decode(kind, a_bits).astype(np.float64)
    b = O.narrow_decode(kind, b_bits).astype(np.float64)
    ref = a @ b
    k = a.shape[-1]
    ulp = 2.0**-8 if kind == "bf16" else 2.0**-11
    return ref, ulp * np.abs(ref) + (k + 2) * 2.0**-24 * (np.abs(a) @ np.abs(b)) + 2.0**-133


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("shape", [(256, 256, 256), (200, 130, 77), (1, 64, 300), (64, 1, 128), (128, 384, 512),
                                   (3, 5, 40)])
def test_narrow_matmul_mfma_within_bound(kind, shape):
    M, N, K = shape
    a, b = finite_bits(kind, (M, K), 10), finite_bits(kind, (K, N), 11)
    c = C.matmul(C.to_device(carrier(kind, a)), C.to_device(carrier(kind, b)))
    got = O.narrow_decode(kind, bits_of(c.numpy())).astype(np.float64)
    ref, bound = _mm_bound(kind, a, b)
    bad = np.abs(got - ref) > bound
    assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], ref[bad][:5])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("b_along_k", [False, True])
@pytest.mark.parametrize("shape", [(128, 256, 192), (256, 128, 64), (384, 256, 320)])
def test_narrow_matmul_whole_tiles(kind, b_along_k, shape):
    """Whole 128 x 128 tiles and whole 64-deep K steps (the two-staging-set
    kernel), B along N (row-major) or along K (a transposed view), odd and
    even step counts: within the same bound as every other product."""
    M, N, K = shape
    a, b = finite_bits(kind, (M, K), 20), finite_bits(kind, (K, N), 21)
    da = C.to_device(carrier(kind, a))
    if b_along_k:
        dbt = C.to_device(carrier(kind, np.ascontiguousarray(b.T)))
        db = dbt.view((K, N), (1, K))
    else:
        db = C.to_device(carrier(kind, b))
    c = C.matmul(da, db)
    got = O.narrow_decode(kind, bits_of(c.numpy())).astype(np.float64)
    ref, bound = _mm_bound(kind, a, b)
    bad = np.abs(got - ref) > bound
    assert not bad.any(), (np.argwhere(bad)[:5], got[bad][:5], ref[bad][:5])


@pytest.mark.parametrize("kind", KINDS)
def test_narrow_matmul_whole_tiles_batched(kind):
    """A batch of whole-tile products against one broadcast B (batch stride 0)."""
    a, b = finite_bits(kind, (3, 128, 256), 22), finite_bits(kind, (256, 128), 23)
    c = C.matmul(C.to_device(carrier(kind, a)), C.to_device(carrier(kind, b)))
    got = O.narrow_decode(kind, bits_of(c.numpy())).astype(np.float64)
    ref, bound = _mm_bound(kind, a, b)
    assert np.all(np.abs(got - ref) <= bound)


@pytest.mark.parametrize("kind", KINDS)
def test_narrow_matmul_transposed_and_batched(kind):
    """Transposed operands (stride swaps), a broadcast batch axis, and the
    element-by-element staging of a misaligned view."""
    rng_a = finite_bits(kind, (2, 64, 96), 12)
    rng_b = finite_bits(kind, (80, 96), 13)  # used as b^T: [96, 80] with strides (1, 96)
    da, db = C.to_device(carrier(kind, rng_a)), C.to_device(carrier(kind, rng_b))
    bt = db.view((96, 80), (1, 96))
    c = C.matmul(da, bt)
    got = O.narrow_decode(kind, bits_of(c.numpy())).astype(np.float64)
    ref, bound = _mm_bound(kind, rng_a, np.ascontiguousarray(rng_b.T))
    assert np.all(np.abs(got - ref) <= bound)
    # a misaligned A view: one element in
    flat = finite_bits(kind, 96 * 64 + 1, 14)
    dflat = C.to_device(carrier(kind, flat))
    av = dflat.view((96, 64), (64, 1), 1)
    bb = finite_bits(kind, (64, 48), 15)
    c2 = C.matmul(av, C.to_device(carrier(kind, bb)))
    got2 = O.narrow_decode(kind, bits_of(c2.numpy())).astype(np.float64)
    ref2, bound2 = _mm_bound(kind, flat[1:].reshape(96, 64), bb)
    assert np.all(np.abs(got2 - ref2) <= bound2)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("shape", [(64, 48, 80), (130, 70, 300), (1, 33, 65)])
def test_narrow_matmul_exact_bit_exact(kind, shape):
    M, N, K = shape
    a, b = random_bits(kind, (M, K), 16), random_bits(kind, (K, N), 17)
    c = C.matmul(C.to_device(carrier(kind, a)), C.to_device(carrier(kind, b)), exact=True)
    want = O.narrow_matmul(kind, a, b)
    assert np.array_equal(bits_of(c.numpy()), want)


@pytest.mark.parametrize("kind", KINDS)
def test_narrow_linear_epilogue_unsupported(kind):
    a = C.to_device(carrier(kind, random_bits(kind, (4, 4), 18)))
    with pytest.raises(C.ChelisError, match="no fused epilogue"):
        C.linear(a, a, act="relu")

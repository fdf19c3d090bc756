"""GPU parity of the matmul dispatch against the C oracle's canonical-tree
matmul (crates/chelis-backend-c/src/emit.rs:8431-8560).

Bar: the canonical-tree kernels (short K, GEMV, skinny, and every shape
under the exact flag) are bit-exact; the MFMA tile kernels differ from the
tree by rounding only and must stay within the north star's tolerances:
normwise ||c - ref||_inf / ||ref||_inf <= 1e-5 for f32 and <= 1e-10 for f64,
and the same bound elementwise relative wherever |ref| >= rms(ref) (below
that, cancellation makes the relative error of any summation order grow as
rms/|ref|; the normwise bound covers those entries).
"""
import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = {np.float32: 1e-5, np.float64: 1e-10}


def setup_module(_m):
    O.build()


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def first_diff(a, b):
    bad = np.argwhere(~((a == b) | (np.isnan(a) & np.isnan(b))))
    return f"{len(bad)} differ; first {bad[:3].tolist()}"


def dev_view(host_full, rows, cols, transposed):
    """(device tensor keeping storage alive, device view, numpy view) of a
    rows x cols operand, stored transposed when asked."""
    if transposed:
        base = np.ascontiguousarray(host_full.T)
        d = C.to_device(base)
        return d, d.view((rows, cols), (1, rows)), base.T
    d = C.to_device(np.ascontiguousarray(host_full))
    return d, d, host_full


def rand(rng, shape, dtype):
    return rng.uniform(-1, 1, shape).astype(dtype)


def check_close(c, ref, dtype):
    tol = TOL[dtype]
    scale = np.abs(ref).max()
    assert np.abs(c - ref).max() <= tol * scale, ("normwise", np.abs(c - ref).max() / scale)
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    big = np.abs(ref) >= rms
    rel = np.abs(c - ref)[big] / np.abs(ref)[big]
    assert rel.max() <= tol, ("elementwise", rel.max())


TREE_CASES = [
    # (M, N, K, a transposed, b transposed) - family chosen by the dispatch
    (37, 50, 1, False, False),      # short K
    (64, 33, 17, True, False),      # short K
    (128, 512, 10, False, True),    # short K (the MLP's g_z2 . W2^T form)
    (8192, 1, 32, False, False),    # short K, vector reads of A and B (the linreg X . w form)
    (64, 20, 24, False, True),      # short K, vector runs and a zero-padded tail
    (99, 2, 7, False, True),        # short K, odd row stride (scalar reads)
    (300, 1, 1000, False, False),   # GEMV
    (300, 1, 1000, True, False),    # GEMV, transposed A (linreg X^T r form)
    (1, 257, 4097, False, False),   # row vector times matrix
    (3, 1, 131072, False, False),   # GEMV: f64 exactly 256 segments (shallow carry stack)
    (2, 1, 131073, False, False),   # one leaf more: the deep carry stack
    (100, 10, 3000, False, False),  # skinny (the MLP's d . W2 form)
    (512, 10, 1024, True, False),   # skinny, transposed A (d^T . g_z2)
    (50, 13, 513, False, True),     # skinny, transposed B
    # column-panel kernel (narrow side <= 64 on the lanes)
    (70, 64, 640, False, False),    # N = 64, ragged row groups, K a multiple of the 64-leaf chunk
    (40, 300, 700, False, False),   # M is the narrow side: operand roles swapped
    (33, 129, 777, True, True),     # swapped, both transposed
    (900, 48, 5000, False, False),  # several aligned K blocks and a partial last chunk
    (20, 5, 2049, False, True),     # small product: one K block of 2049 leaves
    (30, 7, 9000, True, False),     # small product, K past one deep block: three blocks and a combine
    (32, 1, 8192, True, False),     # GEMV, A stored along the outputs (linreg X^T r): outputs on the lanes
    (64, 1, 1000, True, False),     # the same with a full 64-lane panel
    (1, 48, 5000, False, False),    # row vector times a row-major matrix: outputs on the lanes
    (1, 64, 33, False, False),      # the same, one partial chunk
    (4, 1, 262145, True, False),    # linreg X^T r form, K past 255 blocks of 512: the deep block-total join
    (3, 5, 300000, False, False),   # panel, 586 block totals
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("case", TREE_CASES)
def test_tree_kernels_bit_exact(case, dtype):
    M, N, K, ta, tb = case
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    a, b = rand(rng, (M, K), dtype), rand(rng, (K, N), dtype)
    _da, va, na = dev_view(a, M, K, ta)
    _db, vb, nb = dev_view(b, K, N, tb)
    # a narrow side of 16..64 is an MFMA shape; the exact flag keeps it on
    # the canonical tree (the column-panel kernel)
    exact = K > 32 and min(M, N) >= 16
    c = C.matmul(va, vb, exact=exact).numpy()
    ref = O.matmul(na, nb)
    assert bits_equal(c, ref), first_diff(c, ref)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_exact_flag_on_dense_shape(dtype):
    rng = np.random.default_rng(21)
    a, b = rand(rng, (200, 300), dtype), rand(rng, (300, 130), dtype)
    c = C.matmul(C.to_device(a), C.to_device(b), exact=True).numpy()
    assert bits_equal(c, O.matmul(a, b))


def test_f64_skinny_band_tolerance_and_exact_flag():
    """f64 with 16 <= min(M, N) <= 64 runs on the MFMA tiles within the 1e-10
    GEMM tolerance; the exact flag keeps it on the canonical tree."""
    rng = np.random.default_rng(22)
    a, b = rand(rng, (700, 900), np.float64), rand(rng, (900, 64), np.float64)
    ref = O.matmul(a, b)
    c = C.matmul(C.to_device(a), C.to_device(b)).numpy()
    check_close(c, ref, np.float64)
    assert bits_equal(C.matmul(C.to_device(a), C.to_device(b), exact=True).numpy(), ref)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_exact_flag_narrow_f32_and_batched_panel(dtype):
    """A batch of narrow products (the panel kernel over blockIdx.z), with a
    broadcast batch operand, and the exact flag on a 16 <= N <= 64 shape."""
    rng = np.random.default_rng(23)
    a, b = rand(rng, (3, 150, 600), dtype), rand(rng, (600, 40), dtype)
    c = C.matmul(C.to_device(a), C.to_device(b), exact=True).numpy()
    assert c.shape == (3, 150, 40)
    for i in range(3):
        assert bits_equal(c[i], O.matmul(a[i], b)), i


def test_empty_contraction_is_positive_zero():
    a = C.empty((5, 0), np.float32)
    b = C.empty((0, 7), np.float32)
    c = C.matmul(a, b).numpy()
    assert c.shape == (5, 7) and bits_equal(c, np.zeros((5, 7), np.float32))


def test_special_values_tree():
    """Signed zeros, infinities, NaN and cancellation through the exact tree."""
    a = np.array([[1e8, 1.0, -1e8, 1.0], [-0.0, -0.0, -0.0, -0.0], [np.inf, 1.0, -np.inf, 0.0],
                  [np.nan, 0.0, 0.0, 0.0], [1e-38, 1e-38, -1e-38, 1e-45]], np.float32)
    b = np.array([[1.0], [1.0], [1.0], [1.0]], np.float32)
    c = C.matmul(C.to_device(a), C.to_device(b)).numpy()
    ref = O.matmul(a, b)
    assert bits_equal(c, ref), (c.ravel(), ref.ravel())


def test_config_3d_gemv_bit_exact():
    rng = np.random.default_rng(26)
    A = rng.uniform(-1, 1, (8192, 8192))
    x = np.random.default_rng(27).uniform(-1, 1, 8192)
    y = C.matmul(C.to_device(A), C.to_device(x)).numpy()
    ref = O.matmul(A, x.reshape(-1, 1)).ravel()
    assert y.shape == (8192,) and bits_equal(y, ref)


def test_config_3c_skinny():
    """Config 3c at full size: the default (MFMA, split-K) result within the
    1e-10 f64 GEMM tolerance, the exact flag's bit-exact."""
    A = np.random.default_rng(24).uniform(-1, 1, (8192, 4096))
    B = np.random.default_rng(25).uniform(-1, 1, (4096, 64))
    ref = O.matmul(A, B)
    dA, dB = C.to_device(A), C.to_device(B)
    check_close(C.matmul(dA, dB).numpy(), ref, np.float64)
    assert bits_equal(C.matmul(dA, dB, exact=True).numpy(), ref)


MFMA_CASES = [
    (128, 128, 128, False, False),
    (300, 260, 500, False, False),
    (1000, 777, 999, True, False),
    (257, 300, 129, False, True),
    (256, 512, 64, True, True),
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("case", MFMA_CASES)
def test_mfma_within_tolerance(case, dtype):
    M, N, K, ta, tb = case
    rng = np.random.default_rng(M + N + K)
    a, b = rand(rng, (M, K), dtype), rand(rng, (K, N), dtype)
    _da, va, na = dev_view(a, M, K, ta)
    _db, vb, nb = dev_view(b, K, N, tb)
    c = C.matmul(va, vb).numpy()
    check_close(c, O.matmul(na, nb), dtype)


def test_batched_broadcast_attention_form():
    """[2,3,S,d] . [2,3,d,S]^T-style batched products with a broadcast batch axis."""
    rng = np.random.default_rng(31)
    q = rand(rng, (2, 3, 96, 64), np.float32)
    k = rand(rng, (2, 1, 96, 64), np.float32)
    dq, dk = C.to_device(q), C.to_device(k)
    kt = dk.view((2, 1, 64, 96), (96 * 64, 96 * 64, 1, 64))  # k^T without a copy
    s = C.matmul(dq, kt).numpy()
    assert s.shape == (2, 3, 96, 96)
    for i in range(2):
        for h in range(3):
            check_close(s[i, h], O.matmul(q[i, h], np.ascontiguousarray(k[i, 0].T)), np.float32)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_config_3ab_4096_cube_every_row(dtype):
    """Configs 3a / 3b at full size: the canonical-tree product (the exact
    flag) equals the oracle on sampled rows, and the default MFMA product is
    within the normwise bar of it on every row, and elementwise on the
    sampled rows. Over all 16.7M binary32 outputs the MFMA tiles' sequential
    accumulation along K (error growing as sqrt(K / 4) roundings) leaves the
    worst entry at about 1.2e-5 relative: measured here as at most 2e-5, with
    at least 99.999 % of the entries >= rms within 1e-5."""
    seeds = (20, 21) if dtype == np.float32 else (22, 23)
    A = np.random.default_rng(seeds[0]).uniform(-1, 1, (4096, 4096)).astype(dtype)
    B = np.random.default_rng(seeds[1]).uniform(-1, 1, (4096, 4096)).astype(dtype)
    dA, dB = C.to_device(A), C.to_device(B)
    c = C.matmul(dA, dB).numpy()
    rows = np.random.default_rng(0).choice(4096, 48, replace=False)
    rows = np.concatenate([[0, 127, 128, 4095], rows])
    tree = C.matmul(dA, dB, exact=True).numpy()
    # the canonical-tree kernels are the oracle's bits on the sampled rows
    assert bits_equal(tree[rows], O.matmul(np.ascontiguousarray(A[rows]), B))
    check_close(c[rows], tree[rows], dtype)
    tol = TOL[dtype]
    err = np.abs(c.astype(np.float64) - tree)
    assert err.max() <= tol * np.abs(tree).max()
    big = np.abs(tree) >= np.sqrt(np.mean(tree.astype(np.float64) ** 2))
    rel = err[big] / np.abs(tree[big])
    if dtype == np.float64:
        assert rel.max() <= tol
    else:
        assert rel.max() <= 2 * tol and np.mean(rel > tol) <= 1e-5, (rel.max(), np.mean(rel > tol))


@pytest.mark.parametrize("act", [None, "relu", "gelu"])
def test_linear_epilogue_bit_exact_on_tree_path(act):
    """bias, activation and residual fused after a skinny (tree) product equal
    the unfused graph bit for bit."""
    rng = np.random.default_rng(41)
    x, w = rand(rng, (256, 512), np.float32), rand(rng, (512, 10), np.float32)
    bias, res = rand(rng, (10,), np.float32), rand(rng, (256, 10), np.float32)
    # the GELU graph bit for bit is the exact mode's (the default mode's
    # binary32 GELU is the direct evaluation, within 1e-6 of it)
    prev = C.set_exact(act == "gelu")
    try:
        c = C.linear(C.to_device(x), C.to_device(w), C.to_device(bias), act, C.to_device(res)).numpy()
    finally:
        C.set_exact(prev)
    v = (O.matmul(x, w) + bias).astype(np.float32)
    if act == "relu":
        v = O.relu(v)
    elif act == "gelu":
        v = O.gelu(v)
    v = (res + v).astype(np.float32)
    assert bits_equal(c, v), first_diff(c, v)
    if act == "gelu":
        d = C.linear(C.to_device(x), C.to_device(w), C.to_device(bias), act, C.to_device(res)).numpy()
        assert np.all(np.abs(d.astype(np.float64) - v) <= 1e-6 * np.abs(v) + 1e-6 * np.abs(res).max())


@pytest.mark.parametrize("exact", [True, False])
def test_gelu_epilogue_on_the_mfma_tiles(exact):
    """The GELU epilogue of a dense binary32 product (the FFN1 form) against
    the exact GELU graph (C.gelu in the exact mode) of the same product
    computed in the same mode without the activation (the same
    accumulation): bit for bit in the exact mode; the default mode's
    direct evaluation within 1e-6 of it."""
    rng = np.random.default_rng(44)
    x, w = rand(rng, (512, 256), np.float32), rand(rng, (256, 384), np.float32)
    bias = rand(rng, (384,), np.float32)
    dx, dw, db = C.to_device(x), C.to_device(w), C.to_device(bias)
    prev = C.set_exact(exact)
    try:
        c = C.linear(dx, dw, db, "gelu").numpy()
        pre = C.linear(dx, dw, db, None)
    finally:
        C.set_exact(prev)
    prev = C.set_exact(True)
    try:
        ref = C.gelu(pre).numpy()
    finally:
        C.set_exact(prev)
    if exact:
        assert bits_equal(c, ref), first_diff(c, ref)
    else:
        assert np.all(np.abs(c.astype(np.float64) - ref) <= 1e-6 * np.abs(ref) + 2.0 ** -146)


def test_linear_epilogue_on_swapped_panel_path():
    """A narrow M (< 16) with N > 64 runs as c^T = w^T x^T; the bias and
    residual must still follow the output's own axes."""
    rng = np.random.default_rng(43)
    x, w = rand(rng, (8, 300), np.float32), rand(rng, (300, 500), np.float32)
    bias, res = rand(rng, (500,), np.float32), rand(rng, (8, 500), np.float32)
    c = C.linear(C.to_device(x), C.to_device(w), C.to_device(bias), "relu", C.to_device(res)).numpy()
    v = (res + O.relu((O.matmul(x, w) + bias).astype(np.float32))).astype(np.float32)
    assert bits_equal(c, v), first_diff(c, v)


def test_linear_per_batch_bias():
    """A stack of projections: a broadcast over the batch, b and bias with one
    entry per batch ([batch, K, N] and [batch, N]), bit-exact on the tree
    path (the exact flag: an f64 narrow side of 40 is an MFMA shape by
    default); and the same on an MFMA shape within tolerance."""
    rng = np.random.default_rng(44)
    x = rand(rng, (96, 200), np.float64)
    w, bias = rand(rng, (3, 200, 40), np.float64), rand(rng, (3, 40), np.float64)
    dx = C.to_device(x)
    x3 = dx.view((3, 96, 200), (0, 200, 1))
    c = C.linear(x3, C.to_device(w), C.to_device(bias), exact=True).numpy()
    for j in range(3):
        assert bits_equal(c[j], O.matmul(x, w[j]) + bias[j]), j
    xf = rand(rng, (256, 128), np.float32)
    wf, bf = rand(rng, (3, 128, 192), np.float32), rand(rng, (3, 192), np.float32)
    cf = C.linear(C.to_device(xf).view((3, 256, 128), (0, 128, 1)), C.to_device(wf), C.to_device(bf)).numpy()
    for j in range(3):
        check_close(cf[j], (O.matmul(xf, wf[j]) + bf[j]).astype(np.float32), np.float32)


def test_linear_epilogue_on_mfma_path():
    rng = np.random.default_rng(42)
    x, w = rand(rng, (512, 256), np.float32), rand(rng, (256, 384), np.float32)
    bias = rand(rng, (384,), np.float32)
    c = C.linear(C.to_device(x), C.to_device(w), C.to_device(bias), "relu").numpy()
    check_close(c, O.relu((O.matmul(x, w) + bias).astype(np.float32)), np.float32)


# Products whose tiles do not fill the chip and whose K runs long split K into
# slices summed in slice order by a combine pass (still an MFMA-tolerance path).
SPLIT_CASES = [
    (784, 512, 1024, True, False),  # the MLP's x^T g
    (100, 130, 3001, False, True),  # ragged last slice
    (96, 200, 8192, True, True),    # 16 slices
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("case", SPLIT_CASES)
def test_split_k_within_tolerance(case, dtype):
    M, N, K, ta, tb = case
    rng = np.random.default_rng(M * 7 + N + K)
    a, b = rand(rng, (M, K), dtype), rand(rng, (K, N), dtype)
    _da, va, na = dev_view(a, M, K, ta)
    _db, vb, nb = dev_view(b, K, N, tb)
    c = C.matmul(va, vb).numpy()
    check_close(c, O.matmul(na, nb), dtype)


def test_split_k_batched_with_epilogue():
    """Per-batch bias, GELU and residual applied once, after the slices are
    summed; a broadcast batch operand."""
    rng = np.random.default_rng(45)
    x = rand(rng, (3, 96, 1500), np.float64)
    w, bias = rand(rng, (1500, 100), np.float64), rand(rng, (3, 100), np.float64)
    res = rand(rng, (3, 96, 100), np.float64)
    dw = C.to_device(w)
    c = C.linear(C.to_device(x), dw.view((3, 1500, 100), (0, 100, 1)), C.to_device(bias), "gelu",
                 C.to_device(res)).numpy()
    for j in range(3):
        v = res[j] + O.gelu(O.matmul(x[j], w) + bias[j])
        check_close(c[j], v, np.float64)


# A narrow side of 16..64 on the MFMA tiles (the 64-tile, K split over
# workgroups when the tiles cannot fill the chip): ragged edges, strided and
# misaligned operands, batches and epilogues.
SKINNY_CASES = [
    # (M, N, K, b transposed, a row offset in elements)
    (8192, 64, 4096, False, 0),  # config 3c's shape (two K slices)
    (1000, 33, 1001, False, 0),  # ragged rows, columns and K (a partial last chunk)
    (37, 16, 5000, True, 0),     # few rows: many K slices; B stored along K
    (512, 48, 70, False, 0),     # K of 4.4 chunks: waves with 2 and 1 chunks
    (300, 64, 640, False, 1),    # A rows start off the 16-byte grid: element loads
    (64, 20, 33, False, 0),      # K of 3 chunks, most waves idle
]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("case", SKINNY_CASES)
def test_skinny_within_tolerance(case, dtype):
    M, N, K, tb, off = case
    rng = np.random.default_rng(M + 3 * N + K)
    a, b = rand(rng, (M, K), dtype), rand(rng, (K, N), dtype)
    if off:
        # rows of K + 1 elements starting at element `off`: a strided view
        # whose rows are not 16-byte aligned
        buf = np.zeros(M * (K + 1) + off, dtype)
        buf[off:].reshape(M, K + 1)[:, :K] = a
        d = C.to_device(buf)
        va = d.view((M, K), (K + 1, 1), off)
    else:
        _d, va, _n = dev_view(a, M, K, False)
    _db, vb, nb = dev_view(b, K, N, tb)
    c = C.matmul(va, vb).numpy()
    check_close(c, O.matmul(a, nb), dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("act", [None, "relu", "gelu"])
def test_skinny_batched_epilogue(dtype, act):
    """A broadcast batch (B shared), per-batch bias, activation and residual
    on a narrow product: applied in the tile kernel (one slice) or in the
    split-K combine pass."""
    rng = np.random.default_rng(46)
    for M, K in ((2048, 256), (96, 3000)):
        x = rand(rng, (2, M, K), dtype)
        w, bias = rand(rng, (K, 40), dtype), rand(rng, (2, 40), dtype)
        res = rand(rng, (2, M, 40), dtype)
        dw = C.to_device(w)
        c = C.linear(C.to_device(x), dw.view((2, K, 40), (0, 40, 1)), C.to_device(bias), act,
                     C.to_device(res)).numpy()
        for j in range(2):
            v = (O.matmul(x[j], w) + bias[j]).astype(dtype)
            if act == "relu":
                # the oracle's relu is binary32 only; max(v, +0) is exact
                v = O.relu(v) if dtype == np.float32 else np.where(v < 0, 0.0, v)
            elif act == "gelu":
                v = O.gelu(v)
            check_close(c[j], (res[j] + v).astype(dtype), dtype)


def test_skinny_repeatable():
    """The same inputs give the same bits on every call (fixed tile and
    slice order)."""
    rng = np.random.default_rng(47)
    a, b = rand(rng, (4000, 3000), np.float64), rand(rng, (3000, 64), np.float64)
    da, db = C.to_device(a), C.to_device(b)
    c0 = C.matmul(da, db).numpy()
    for _ in range(3):
        assert bits_equal(C.matmul(da, db).numpy(), c0)


@pytest.mark.parametrize("act", [None, "relu"])
def test_batched_projection_shape_with_per_batch_bias(act):
    """Three [4096 x 1024] x [1024 x 1024] f32 products with per-batch bias
    (the transformer's Q/K/V shape: 768 128-tiles, a round and a half of the
    resident workgroups): sampled rows of every batch against float64."""
    rng = np.random.default_rng(46)
    x = rand(rng, (3, 4096, 1024), np.float32)
    w = rand(rng, (3, 1024, 1024), np.float32)
    bias = rand(rng, (3, 1024), np.float32)
    c = C.linear(C.to_device(x), C.to_device(w), C.to_device(bias), act).numpy()
    rows = rng.choice(4096, 48, replace=False)
    for j in range(3):
        ref = x[j][rows].astype(np.float64) @ w[j].astype(np.float64) + bias[j]
        if act == "relu":
            ref = np.maximum(ref, 0.0)
        got = c[j][rows].astype(np.float64)
        assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-5, j

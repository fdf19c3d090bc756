"""GPU parity of the configuration programs (include/chelis_programs.h)
against the C oracle's restated programs (oracle/chelis_oracle.c).

Bar:
  * linreg_step (config 1, f64): every matmul of the program is on the
    canonical-tree path (short K and GEMV), every reduction is the tree, so
    grad and loss are bit-exact at the config's full size.
  * mlp_train_step (config 5, f32): with the exact-matmul mode every result
    is bit-exact (canonical-tree products, correctly rounded exp and log
    leaves); with the default MFMA dispatch, within 1e-5 relative normwise
    (the f32 tolerance).
  * transformer_block (config 4, f32, full size): within 1e-5 relative
    normwise (MFMA products; every f32 leaf correctly rounded).
"""
import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def setup_module(_m):
    O.build()


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def normwise(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-300))


def linreg_inputs(n=8192, d=32):
    X = np.random.default_rng(1).standard_normal((n, d))
    w = np.random.default_rng(2).standard_normal(d)
    y = X @ w + np.random.default_rng(3).normal(0, 0.01, n)
    return X, w, y


def test_linreg_step_config1_bit_exact():
    X, w, y = linreg_inputs()
    grad_ref, loss_ref = O.linreg_step(X, w, y)
    ins = [C.to_device(a) for a in (X, w, y)]
    grad, loss = C.empty((32,), np.float64), C.empty((), np.float64)
    C.program("linreg_step", ins, [grad, loss])
    assert bits_equal(grad.numpy(), grad_ref)
    assert bits_equal(loss.numpy(), np.float64(loss_ref))


@pytest.mark.parametrize("n,d", [(1, 1), (63, 2), (65, 3), (8193, 32), (4096 * 64, 8), (4096 * 64 + 1, 4), (300, 33)])
def test_linreg_step_shapes_bit_exact(n, d):
    """Ragged row blocks, every register-tree width, the largest row count
    the two-launch step takes (4096 blocks of 64 rows) and the first past it,
    and d = 33 (past the short contraction): all bit-exact."""
    X, w, y = linreg_inputs(n, d)
    grad_ref, loss_ref = O.linreg_step(X, w, y)
    ins = [C.to_device(a) for a in (X, w, y)]
    grad, loss = C.empty((d,), np.float64), C.empty((), np.float64)
    C.program("linreg_step", ins, [grad, loss])
    assert bits_equal(grad.numpy(), grad_ref)
    assert bits_equal(loss.numpy(), np.float64(loss_ref))


def test_linreg_step_device_entry_allocates_outputs():
    X, w, y = linreg_inputs(1000, 7)
    grad_ref, loss_ref = O.linreg_step(X, w, y)
    grad, loss = C.device_entry("linreg_step", [C.to_device(a) for a in (X, w, y)], 2)
    assert grad.shape == (7,) and loss.shape == ()
    assert bits_equal(grad.numpy(), grad_ref) and bits_equal(loss.numpy(), np.float64(loss_ref))


def mlp_inputs(B=1024, I=784, H=512, O_=10):
    x = np.random.default_rng(40).uniform(0, 1, (B, I)).astype(np.float32)
    labels = np.random.default_rng(41).integers(0, O_, B)
    onehot = np.eye(O_, dtype=np.float32)[labels]
    w1 = (np.random.default_rng(42).standard_normal((I, H)) * np.sqrt(2 / I)).astype(np.float32)
    w2 = (np.random.default_rng(43).standard_normal((H, O_)) * np.sqrt(2 / H)).astype(np.float32)
    b1, b2 = np.zeros(H, np.float32), np.zeros(O_, np.float32)
    return x, onehot, w1, b1, w2, b2


def run_mlp(args, key):
    x, onehot, w1, b1, w2, b2 = args
    ins = [C.to_device(a) for a in args] + [C.key_tensor(key)]
    outs = [C.empty((), np.float32), C.empty(w1.shape, np.float32), C.empty(b1.shape, np.float32),
            C.empty(w2.shape, np.float32), C.empty(b2.shape, np.float32)]
    C.program("mlp_train_step", ins, outs)
    return [o.numpy() for o in outs]


@pytest.mark.parametrize("exact", [True, False])
def test_mlp_train_step_config5(exact):
    args = mlp_inputs()
    key = 44  # key_from_seed(44): the seed's bits
    ref = O.mlp_train_step(*args, key, np.float32(0.1), np.float32(0.01))
    prev = C.set_exact_matmul(exact)
    try:
        got = run_mlp(args, key)
    finally:
        C.set_exact_matmul(prev)
    if exact:
        for g, r, name in zip(got, ref, ("loss", "w1", "b1", "w2", "b2")):
            assert np.array_equal(np.asarray(g, np.float32).view(np.uint32),
                                  np.asarray(r, np.float32).view(np.uint32)), (name, normwise(g, r))
        return
    loss_ulps = abs(int(np.float32(got[0]).view(np.int32)) - int(np.float32(ref[0]).view(np.int32)))
    assert loss_ulps <= 64, (got[0], ref[0])
    for g, r, name in zip(got[1:], ref[1:], ("w1", "b1", "w2", "b2")):
        err = normwise(g, r)
        assert err <= 1e-5, (name, err)


@pytest.mark.parametrize("B,I,H,O_", [
    (1, 8, 5, 1),         # one row, one class, a partial lane run
    (100, 50, 70, 3),     # ragged row blocks, H past one 64-unit group, scalar rows (H % 4 != 0)
    (65, 33, 1024, 16),   # the widest fused head (16 units per lane, 16 classes)
    (130, 40, 96, 7),     # three row blocks
    (64, 16, 1100, 4),    # H past the fused head: the unfused launches
    (64, 16, 64, 17),     # 17 classes: the unfused launches
])
def test_mlp_train_step_shapes_bit_exact(B, I, H, O_):
    """Under the exact flag every launch of the step is a canonical-tree or
    correctly rounded primitive, so each output is bit-identical to the C
    oracle; biases are nonzero here so the bias steps are checked too."""
    x, onehot, w1, b1, w2, b2 = mlp_inputs(B, I, H, O_)
    b1 = np.random.default_rng(44).standard_normal(H).astype(np.float32) * 0.1
    b2 = np.random.default_rng(45).standard_normal(O_).astype(np.float32) * 0.1
    args = (x, onehot, w1, b1, w2, b2)
    ref = O.mlp_train_step(*args, 7, np.float32(0.1), np.float32(0.01))
    prev = C.set_exact_matmul(True)
    try:
        got = run_mlp(args, 7)
    finally:
        C.set_exact_matmul(prev)
    for g, r, name in zip(got, ref, ("loss", "w1", "b1", "w2", "b2")):
        assert np.array_equal(np.asarray(g, np.float32).view(np.uint32),
                              np.asarray(r, np.float32).view(np.uint32)), (name, normwise(g, r))


def test_mlp_train_step_updates_match_in_exact_mode():
    """The parameter deltas w' - w (lr * gradient) agree to 1e-5 relative
    normwise on every parameter, a much tighter check than on w' itself."""
    args = mlp_inputs(256, 784, 128, 10)
    ref = O.mlp_train_step(*args, 44, np.float32(0.1), np.float32(0.01))
    prev = C.set_exact_matmul(True)
    try:
        got = run_mlp(args, 44)
    finally:
        C.set_exact_matmul(prev)
    for i, p in enumerate((args[2], args[3], args[4], args[5])):
        d_got = got[i + 1].astype(np.float64) - p
        d_ref = ref[i + 1].astype(np.float64) - p
        assert normwise(d_got, d_ref) <= 1e-5, i


def transformer_inputs(B=8, S=512, D=1024, F=4096):
    x = np.random.default_rng(30).standard_normal((B, S, D)).astype(np.float32)
    p = {}
    seeds = iter(range(31, 37))
    for name, shape in (("wq", (D, D)), ("wk", (D, D)), ("wv", (D, D)), ("wo", (D, D)), ("w1", (D, F)),
                        ("w2", (F, D))):
        p[name] = (np.random.default_rng(next(seeds)).standard_normal(shape) * 0.02).astype(np.float32)
    for name, n in (("bq", D), ("bk", D), ("bv", D), ("bo", D), ("b1", F), ("b2", D), ("ln1_b", D), ("ln2_b", D)):
        p[name] = np.zeros(n, np.float32)
    p["ln1_g"] = np.ones(D, np.float32)
    p["ln2_g"] = np.ones(D, np.float32)
    return x, p


@pytest.mark.parametrize("size", ["small", "config4"])
def test_transformer_block(size):
    dims = dict(B=2, S=128, D=256, F=1024) if size == "small" else {}
    x, p = transformer_inputs(**dims)
    heads = x.shape[2] // 64
    ref = O.transformer_block(x, p, heads)
    ins = [C.to_device(x)] + [C.to_device(p[k]) for k in O.TRANSFORMER_PARAMS]
    y = C.empty(x.shape, np.float32)
    C.program("transformer_block", ins, [y])
    assert normwise(y.numpy(), ref) <= 1e-5
    # elementwise: every output within 1e-5 of its own magnitude, with an
    # absolute floor of 1e-5 of the output's rms (measured at config 4:
    # 2.7e-6 at worst in that metric, 4.4e-6 absolute)
    err = np.abs(y.numpy().astype(np.float64) - ref)
    floor = float(np.sqrt(np.mean(ref ** 2)))
    assert np.all(err <= 1e-5 * (np.abs(ref) + floor)), float((err / (np.abs(ref) + floor)).max())


def test_transformer_block_device_entry():
    x, p = transformer_inputs(B=1, S=64, D=128, F=256)
    ref = O.transformer_block(x, p, 2)
    ins = [C.to_device(x)] + [C.to_device(p[k]) for k in O.TRANSFORMER_PARAMS]
    (y,) = C.device_entry("transformer_block", ins, 1)
    assert y.shape == x.shape and normwise(y.numpy(), ref) <= 1e-5


def test_host_entries_match_the_oracle():
    """The generated host-tensor entries {f}(chelis_tensor **, ...): host
    arrays in, fresh host tensors out, the same results as the device form."""
    X, w, y = linreg_inputs(2000, 16)
    grad_ref, loss_ref = O.linreg_step(X, w, y)
    grad, loss = C.host_entry("linreg_step", [X, w, y], 2)
    assert grad.shape == (16,) and loss.shape == ()
    assert bits_equal(grad, grad_ref) and bits_equal(loss, np.float64(loss_ref))
    args = mlp_inputs(256, 784, 128, 10)
    ref = O.mlp_train_step(*args, 44, np.float32(0.1), np.float32(0.01))
    prev = C.set_exact_matmul(True)
    try:
        got = C.host_entry("mlp_train_step", list(args) + [("key", 44)], 5)
    finally:
        C.set_exact_matmul(prev)
    for g, r in zip(got, ref):
        assert bits_equal(np.asarray(g, np.float32), np.asarray(r, np.float32))
    x, p = transformer_inputs(B=1, S=64, D=128, F=256)
    (yt,) = C.host_entry("transformer_block", [x] + [p[k] for k in O.TRANSFORMER_PARAMS], 1)
    assert yt.shape == x.shape and normwise(yt, O.transformer_block(x, p, 2)) <= 1e-5


def test_host_entry_count_mismatch_aborts():
    import subprocess
    import sys
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = (f"import sys; sys.path.insert(0, {root!r}); import numpy as np, chelis_amd as C; "
            "C.host_entry('linreg_step', [np.zeros((4, 2)), np.zeros(2)], 2)")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "linreg_step: expected 3 inputs, got 2" in r.stderr

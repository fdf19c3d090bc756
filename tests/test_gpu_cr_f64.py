"""Device check of the correctly rounded binary64 exp (devmath.h exp_fast /
exp_cr_slow) against CORE-MATH, the C backend's libm
(crates/chelis-crmath/csrc/crmath_ffi.c, with the wrapper's NaN
canonicalization), bit for bit:

- 2^24 seeded inputs from five distributions (the whole finite domain,
  log-uniform magnitudes 2^-60 .. 2^9.5, arguments next to k ln2/64, softmax
  arguments in [-40, 0], the subnormal and overflow edges) through a one-step
  fused f64 exp chain;
- every binary64 exp row of the sampled CORE-MATH worst cases
  (tests/golden/binary64_worst_cases.txt, MPFR-derived) and of the canary
  file (specials, NaN payloads, the overflow and underflow thresholds);
- softmax rows built so that x - max equals a negative worst-case input,
  which the softmax kernel's wave-uniform slow pass must round correctly
  (the exact mode's row; the default row is held to 1e-13).
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="module")
def cr(tmp_path_factory):
    O.build()
    so = tmp_path_factory.mktemp("cr64") / "libcr_array.so"
    ref = os.path.join(ROOT, "oracle", "_ref")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-o", str(so),
                    os.path.join(ROOT, "tests", "cpu", "cr_array.c"), f"-L{ref}", "-lcrmath_ref",
                    f"-Wl,-rpath,{ref}"], check=True)
    lib = ctypes.CDLL(str(so))
    lib.cr_check64.restype = ctypes.c_long
    lib.cr_check64.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_long, ctypes.c_void_p, ctypes.c_void_p,
                               ctypes.c_long]
    return lib


def fixture_inputs(name):
    rows = []
    with open(os.path.join(GOLDEN, name)) as f:
        for line in f:
            p = line.split()
            if len(p) >= 4 and p[0] == "exp" and p[1] == "f64":
                rows.append((int(p[2], 16), int(p[3], 16)))
    return np.array([r[0] for r in rows], np.uint64), np.array([r[1] for r in rows], np.uint64)


def random_inputs(n, seed):
    rng = np.random.default_rng(seed)
    k = n // 5
    parts = [
        rng.uniform(-746.0, 711.0, k),
        np.where(rng.random(k) < 0.5, -1, 1) * np.minimum(np.exp2(rng.uniform(-60, 9.5, k)), 700.0),
        rng.integers(-68800, 65500, k) * 0.010830424696249145 + (rng.random(k) - 0.5) * np.exp2(
            -rng.integers(20, 60, k).astype(np.float64)),
        -40.0 * rng.random(k),
        np.where(rng.random(n - 4 * k) < 0.5, rng.uniform(-745.2, -708.2, n - 4 * k),
                 rng.uniform(709.0, 709.8, n - 4 * k)),
    ]
    return np.concatenate(parts)


def device_exp(x):
    out = C.empty(x.shape, np.float64)
    C.fused_elementwise(C.fused_chain([("exp", 0)]), [C.to_device(x)], out)
    return np.ascontiguousarray(out.numpy())


def check(cr, xbits, got, cap=16):
    bad = np.zeros(3 * cap, np.uint64)
    n = cr.cr_check64(0, xbits.ctypes.data, len(xbits), got.view(np.uint64).ctypes.data, bad.ctypes.data, cap)
    return n, [tuple(hex(int(v)) for v in bad[3 * i:3 * i + 3]) for i in range(min(n, cap))]


def test_exp_f64_random_inputs_correctly_rounded(cr):
    x = random_inputs(1 << 24, 2024)
    got = device_exp(x)
    n, bad = check(cr, np.ascontiguousarray(x).view(np.uint64), got)
    assert n == 0, f"{n} mismatches: {bad}"


@pytest.mark.parametrize("name", ["binary64_worst_cases.txt", "crmath_canary.txt"])
def test_exp_f64_fixture_rows(cr, name):
    xin, want = fixture_inputs(name)
    assert len(xin) >= 25
    got = device_exp(xin.view(np.float64)).view(np.uint64)
    assert np.array_equal(got, want), [(hex(a), hex(b), hex(c)) for a, b, c in zip(xin, want, got) if b != c][:8]
    n, bad = check(cr, xin, got.view(np.float64))
    assert n == 0, bad


@pytest.mark.parametrize("n", [777, 4096])
def test_softmax_f64_worst_case_arguments(n):
    """Rows [0, w1, w2, ...] with w the negative worst-case inputs: x - max is
    exactly w, so every flagged element goes through the slow pass."""
    xin, _ = fixture_inputs("binary64_worst_cases.txt")
    w = xin.view(np.float64)
    w = w[w < 0]
    rng = np.random.default_rng(n)
    rows = 64
    x = np.empty((rows, n))
    for r in range(rows):
        x[r] = rng.choice(w, n)
        x[r, rng.integers(0, n)] = 0.0
    ref = O.softmax_rows(x)
    prev = C.set_exact(True)  # the correctly rounded row (the default row's exp is faithful)
    try:
        y = C.softmax(C.to_device(x)).numpy()
    finally:
        C.set_exact(prev)
    assert np.array_equal(y.view(np.uint64), ref.view(np.uint64))
    # the default row on the same arguments: within 1e-13 per element
    y = C.softmax(C.to_device(x)).numpy()
    assert (np.abs(y - ref) <= 1e-13 * np.abs(ref) + 4 * 2.0 ** -1074).all()

"""Exhaustive device check of the binary32 transcendental leaves against
CORE-MATH, and of the binary32 GELU graph against the C oracle (the C backend's libm, crates/chelis-crmath/csrc/crmath_ffi.c,
with the wrapper's NaN canonicalization): every one of the 2^32 binary32
inputs, bit for bit. exp is the correctly rounded expf_cr of devmath.h;
log, erfc and tanh are the binary64 device evaluation rounded once, with
the inputs near a rounding midpoint resolved through the exception tables
of cr_exceptions.h.

Each function takes 16 runs of 2^28 inputs: the device evaluates a run
through a one-step fused chain, the host evaluates CORE-MATH over the same
bit patterns with OpenMP threads and compares.
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
RUN = 1 << 28
OPS = {"exp": 0, "log": 1, "erfc": 2, "tanh": 3}


@pytest.fixture(scope="module")
def cr(tmp_path_factory):
    O.build()
    so = tmp_path_factory.mktemp("cr") / "libcr_array.so"
    ref = os.path.join(ROOT, "oracle", "_ref")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-o", str(so),
                    os.path.join(ROOT, "tests", "cpu", "cr_array.c"), f"-L{ref}", "-lcrmath_ref",
                    f"-Wl,-rpath,{ref}"], check=True)
    lib = ctypes.CDLL(str(so))
    lib.cr_check_run.restype = ctypes.c_long
    lib.cr_check_run.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_long, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_long]
    return lib


def device_run(op, first, n):
    x = (np.arange(n, dtype=np.uint32) + np.uint32(first)).view(np.float32)
    dx = C.to_device(x)
    out = C.empty(x.shape, np.float32)
    C.fused_elementwise(C.fused_chain([(op, 0)]), [dx], out)
    return np.ascontiguousarray(out.numpy()).view(np.uint32)


def mismatches(cr, op, cap=64):
    """(count, [(input, expected, device) bits]) over all 2^32 inputs."""
    total, bad = 0, []
    buf = np.zeros(3 * cap, np.uint32)
    for r in range((1 << 32) // RUN):
        first = r * RUN
        got = device_run(op, first, RUN)
        n = cr.cr_check_run(OPS[op], first, RUN, got.ctypes.data, buf.ctypes.data, cap)
        if n:
            k = min(n, cap)
            bad += [tuple(int(v) for v in buf[3 * i:3 * i + 3]) for i in range(k)]
        total += n
        print(f"{op}: run {r} done, {n} mismatches", flush=True)
    return total, sorted(bad)


@pytest.mark.parametrize("op", ["exp", "log", "erfc", "tanh"])
def test_binary32_leaf_is_correctly_rounded_on_every_input(cr, op):
    n, bad = mismatches(cr, op)
    assert n == 0, f"{n} inputs differ; first {[tuple(hex(v) for v in b) for b in bad[:8]]}"


def test_gelu_f32_matches_the_oracle_on_every_input():
    """GELU in the exact mode over all 2^32 binary32 inputs through the
    unary kernel (whose GELU is the one the GEMM epilogue and the chain
    interpreter inline), bit for bit against the C oracle's restated Phi
    graph with CORE-MATH's erfc and exp leaves: pins the erfc fast path,
    the exp(-th^2) the correction derives from it, their rounding tests and
    fallbacks."""
    O.build()
    total, bad = 0, []
    prev = C.set_exact(True)
    try:
        for r in range((1 << 32) // RUN):
            x = (np.arange(RUN, dtype=np.uint32) + np.uint32(r * RUN)).view(np.float32)
            got = np.ascontiguousarray(C.gelu(C.to_device(x)).numpy()).view(np.uint32)
            ref = np.ascontiguousarray(O.gelu(x)).view(np.uint32)
            diff = np.nonzero(got != ref)[0]
            total += len(diff)
            bad += [(hex(int(x.view(np.uint32)[i])), hex(int(ref[i])), hex(int(got[i]))) for i in diff[:8]]
            print(f"gelu: run {r} done, {len(diff)} mismatches", flush=True)
    finally:
        C.set_exact(prev)
    assert total == 0, f"{total} inputs differ; first {bad[:8]}"


def test_gelu_f32_default_mode_within_its_bound_on_every_input():
    """The binary32 default-mode GELU (gelu_fast_f32) over all 2^32 inputs:
    within 1e-6 relative of the oracle's Phi graph (the north star's bar is
    1e-5) with an absolute floor of 2^-146 for subnormal results, and bit
    for bit on NaN, the infinities, the zeros and below -12.5 (where it
    takes the graph). Reports the largest relative error it saw."""
    O.build()
    worst, worst_x, total = 0.0, None, 0
    for r in range((1 << 32) // RUN):
        bits = np.arange(RUN, dtype=np.uint32) + np.uint32(r * RUN)
        x = bits.view(np.float32)
        got = np.ascontiguousarray(C.gelu(C.to_device(x)).numpy())
        ref = np.ascontiguousarray(O.gelu(x))
        g64, r64 = got.astype(np.float64), ref.astype(np.float64)
        same = got.view(np.uint32) == ref.view(np.uint32)
        special = np.isnan(x) | np.isinf(x) | (x == 0) | (x < -12.5)
        with np.errstate(invalid="ignore", divide="ignore"):
            rel = np.where(same, 0.0, np.abs(g64 - r64) / np.abs(r64))
            close = np.abs(g64 - r64) <= 1e-6 * np.abs(r64) + 2.0 ** -146
        bad = ~same & (special | ~close)
        total += int(bad.sum())
        normal = ~same & ~special & (np.abs(r64) >= 2.0 ** -126)
        if normal.any():
            i = int(np.argmax(np.where(normal, rel, 0.0)))
            if rel[i] > worst:
                worst, worst_x = float(rel[i]), hex(int(bits[i]))
        print(f"gelu default: run {r} done, {int(bad.sum())} outside the bound, worst so far {worst:.3e}", flush=True)
    print(f"gelu default: largest relative error on normal results {worst:.3e} at {worst_x}")
    assert total == 0

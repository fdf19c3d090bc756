"""Host check of the device math in chelis_amd/csrc/devmath.h: the
correctly rounded binary32 exp used by the softmax, GELU and fused-chain
kernels is compared with the CORE-MATH oracle over EVERY binary32 input
(all 2^32 bit patterns: subnormals, infinities, NaNs included), and the
correctly rounded binary64 exp over seeded random inputs and the sampled
CORE-MATH worst cases. The same source is compiled for gfx950, using only
operations that round identically there, so this pins the device results
bit for bit."""
import os
import subprocess

import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_expf_cr_matches_core_math_on_every_binary32(tmp_path):
    O.build()
    exe = tmp_path / "expf_check"
    ref = os.path.join(ROOT, "oracle", "_ref")
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-std=c++17", "-o", str(exe),
                    os.path.join(ROOT, "tests", "cpu", "expf_check.cpp"), f"-L{ref}", "-lcrmath_ref",
                    f"-Wl,-rpath,{ref}"], check=True)
    r = subprocess.run([str(exe), "1"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "checked 4294967296 mismatches 0" in r.stdout


def test_exp_f64_matches_core_math(tmp_path):
    """The correctly rounded binary64 exp: 2 * 10^7 seeded inputs from five
    distributions through exp_cr and through the fixed-point path alone,
    every binary64 exp worst case and canary row (MPFR-derived expected
    bits), against CORE-MATH bit for bit; and the fast path's measured error
    within the 2^-73.7 bound its rounding test assumes."""
    O.build()
    exe = tmp_path / "exp64_check"
    ref = os.path.join(ROOT, "oracle", "_ref")
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-std=c++17", "-o", str(exe),
                    os.path.join(ROOT, "tests", "cpu", "exp64_check.cpp"), f"-L{ref}", "-lcrmath_ref",
                    f"-Wl,-rpath,{ref}"], check=True)
    golden = os.path.join(ROOT, "tests", "golden")
    r = subprocess.run([str(exe), "20000000", "11", os.path.join(golden, "binary64_worst_cases.txt"),
                        os.path.join(golden, "crmath_canary.txt")], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "256 exp f64 rows" in r.stdout and "25 exp f64 rows" in r.stdout
    assert "mismatches 0" in r.stdout
    err = float(r.stdout.split("max-fast-error 2^")[1].split()[0])
    assert err <= -73.7, r.stdout


def test_exp_f64_nonpos_faithful_within_one_ulp(tmp_path):
    """The default binary64 softmax row's exp (exp_nonpos_faithful): over
    2 * 10^7 seeded arguments <= 0 it stays within 1 ulp of CORE-MATH's
    correctly rounded result (1 unit of the least subnormal below 2^-1022),
    and 0, -inf, -746 and NaN give 1, +0, +0 and NaN."""
    O.build()
    exe = tmp_path / "exp64_faithful_check"
    ref = os.path.join(ROOT, "oracle", "_ref")
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-std=c++17", "-o", str(exe),
                    os.path.join(ROOT, "tests", "cpu", "exp64_faithful_check.cpp"), f"-L{ref}", "-lcrmath_ref",
                    f"-Wl,-rpath,{ref}"], check=True)
    r = subprocess.run([str(exe), "20000000", "11"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    ulp = float(r.stdout.split("max-ulp ")[1].split()[0])
    sub = float(r.stdout.split("max-subnormal-units ")[1].split()[0])
    assert ulp <= 1.0 and sub <= 1.0, r.stdout


def test_erfcf_fast_path_matches_core_math_on_every_binary32(tmp_path):
    """The binary32 erfc fast path: every input it does not flag gives
    CORE-MATH's bits (the flagged ones take the fallback, which the device
    test checks over every input)."""
    O.build()
    exe = tmp_path / "erfcf_check"
    ref = os.path.join(ROOT, "oracle", "_ref")
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-std=c++17", "-o", str(exe),
                    os.path.join(ROOT, "tests", "cpu", "erfcf_check.cpp"), f"-L{ref}", "-lcrmath_ref",
                    f"-Wl,-rpath,{ref}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout


def test_quot_f32_matches_ieee_division(tmp_path):
    """The softmax row division v / total through a binary64 reciprocal is
    the correctly rounded binary32 quotient: every binary32 v in (0, 1]
    against 16 totals, and 2^26 random pairs."""
    exe = tmp_path / "div_check"
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-std=c++17", "-o", str(exe),
                    os.path.join(ROOT, "tests", "cpu", "div_check.cpp")], check=True)
    r = subprocess.run([str(exe), "1"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout

"""Host check of the device math in chelis_amd/csrc/devmath.h: the
correctly rounded binary32 exp used by the softmax, GELU and fused-chain
kernels is compared with the CORE-MATH oracle over EVERY binary32 input
(all 2^32 bit patterns: subnormals, infinities, NaNs included). The same
source is compiled for gfx950, using only operations that round identically
there, so this pins the device results bit for bit."""
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

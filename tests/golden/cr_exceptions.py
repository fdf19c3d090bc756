"""Correctly rounded binary32 results at the inputs where the device's
binary64 log and erfc, rounded once to binary32, land on the wrong side of a
rounding midpoint. The inputs were found by the exhaustive device comparison
of tests/test_gpu_cr_f32.py (every binary32 input against CORE-MATH). Here
each value is computed independently with 80-digit decimal arithmetic and
rounded to binary32 by comparing exact distances to the neighbouring binary32
values. Writes cr_exceptions.json beside this script; the device table in
chelis_amd/csrc/chain.h holds the same pairs.

    python tests/golden/cr_exceptions.py
"""
import json
import os
from decimal import Decimal, getcontext

import numpy as np

getcontext().prec = 80
HERE = os.path.dirname(os.path.abspath(__file__))

LOG_INPUTS = [0x3C413D3A, 0x41178FEB, 0x4C5D65A5, 0x65D890D3, 0x6F31A8EC]
ERFC_INPUTS = [0xB76C9F62]


def f32_value(bits: int) -> Decimal:
    return Decimal(float(np.array(bits, np.uint32).view(np.float32)))


def round_to_f32(v: Decimal) -> int:
    """Nearest binary32 to v (no ties occur at these inputs)."""
    f = np.float32(float(v))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    dist = sorted((abs(Decimal(float(c)) - v), int(np.array(c, np.float32).view(np.uint32))) for c in cands)
    assert dist[0][0] != dist[1][0], "tie"
    return dist[0][1]


def atan_inv(n: int) -> Decimal:
    """atan(1/n) by its Taylor series."""
    x = Decimal(1) / n
    x2, term, total, k = x * x, x, x, 1
    eps = Decimal(10) ** -(getcontext().prec + 2)
    while abs(term) > eps:
        term *= -x2
        total += term / (2 * k + 1)
        k += 1
    return total


def pi() -> Decimal:
    return 16 * atan_inv(5) - 4 * atan_inv(239)  # Machin's formula


def erf(x: Decimal) -> Decimal:
    """2/sqrt(pi) * sum_n (-1)^n x^(2n+1) / (n! (2n+1)); |x| small here."""
    x2, term, total, n = x * x, x, x, 0
    eps = Decimal(10) ** -(getcontext().prec + 2)
    while abs(term) > eps:
        n += 1
        term *= -x2 / n
        total += term / (2 * n + 1)
    return 2 / pi().sqrt() * total


def table():
    return {
        "log": [[x, round_to_f32(f32_value(x).ln())] for x in LOG_INPUTS],
        "erfc": [[x, round_to_f32(1 - erf(f32_value(x)))] for x in ERFC_INPUTS],
    }


if __name__ == "__main__":
    t = table()
    with open(os.path.join(HERE, "cr_exceptions.json"), "w") as f:
        json.dump(t, f, indent=1)
    for op, rows in t.items():
        for x, y in rows:
            print(f"{op}: 0x{x:08x} -> 0x{y:08x}")

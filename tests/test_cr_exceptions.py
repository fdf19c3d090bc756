"""The binary32 exception table of the device log and erfc leaves
(chelis_amd/csrc/chain.h): the committed fixture equals the independent
80-digit decimal computation of tests/golden/cr_exceptions.py, equals
CORE-MATH (the C backend's libm), and every pair appears in the device
source."""
import json
import os
import re
import sys

import numpy as np

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import cr_exceptions as G  # noqa: E402

FIXTURE = json.load(open(os.path.join(ROOT, "tests", "golden", "cr_exceptions.json")))


def bits(v) -> int:
    return int(np.array(v, np.float32).view(np.uint32))


def f32(b: int) -> np.float32:
    return np.array(b, np.uint32).view(np.float32)[()]


def test_fixture_matches_decimal_computation():
    assert G.table() == FIXTURE


def test_fixture_matches_core_math():
    O.build()
    L = O.lib()
    for op, fn in (("log", L.orc_logf), ("erfc", L.orc_erfcf)):
        for x, y in FIXTURE[op]:
            assert bits(fn(f32(x))) == y, (op, hex(x))


def test_device_source_holds_every_pair():
    src = open(os.path.join(ROOT, "chelis_amd", "csrc", "chain.h")).read()
    pairs = set(re.findall(r"cr_exception\([^;]*?0x([0-9a-f]{8})u, 0x([0-9a-f]{8})u\)", src))
    want = {(f"{x:08x}", f"{y:08x}") for rows in FIXTURE.values() for x, y in rows}
    assert pairs == want


def test_rounding_helper_on_known_values():
    """round_to_f32 picks the nearest binary32: exact values round to
    themselves, and a value just past a midpoint goes to the far side."""
    from decimal import Decimal
    one = Decimal(1)
    assert G.round_to_f32(one) == 0x3F800000
    ulp = Decimal(2) ** -23
    assert G.round_to_f32(one + ulp / 2 + Decimal(10) ** -40) == 0x3F800001
    assert G.round_to_f32(one + ulp / 2 - Decimal(10) ** -40) == 0x3F800000
    assert G.round_to_f32(Decimal(2).ln()) == bits(np.float32(np.log(np.float64(2))))

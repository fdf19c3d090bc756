"""CPU checks of the C-ABI library: it loads without a GPU, exports every
symbol include/*.h declares, and its host-side runtime (host tensors and
metadata plans) behaves like the reference's, traps included. No device
compute is called here."""
import ctypes
import os
import re
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import chelis_amd as C

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^[A-Za-z_][\w\s\*]*?\b(chelis_\w+)\s*\(", re.M)


def declared_functions():
    names = set()
    for h in os.listdir(os.path.join(ROOT, "include")):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)
        for m in DECL.finditer(text):
            line = text[m.start():text.find("\n", m.start())]
            if line.lstrip().startswith(("typedef", "#", "static")):
                continue
            names.add(m.group(1))
    return names


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", C.LIB_PATH], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}


def test_library_loads_and_exports_every_declared_symbol():
    C.lib()
    declared = declared_functions()
    assert len(declared) > 40, declared
    missing = declared - exported_symbols()
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_python_signatures_cover_only_exported_symbols():
    exported = exported_symbols()
    assert set(C.SIGNATURES) <= exported, sorted(set(C.SIGNATURES) - exported)


def test_build_info():
    assert C.lib().chelis_hip_build_info().decode().startswith("gfx950")


def test_host_tensor_roundtrip_and_views():
    L = C.lib()
    shape = (ctypes.c_int64 * 2)(3, 5)
    t = L.chelis_alloc(2, shape, C.DT_F64)
    assert L.chelis_tensor_rank(t) == 2 and L.chelis_tensor_shape(t, 1) == 5 and L.chelis_tensor_numel(t) == 15
    v = L.chelis_tensor_read_view(t)
    assert v.count == 15 and v.dtype == C.DT_F64
    assert np.ctypeslib.as_array(ctypes.cast(v.data, ctypes.POINTER(ctypes.c_double)), (15,)).sum() == 0
    g = L.chelis_tensor_begin_write(t)
    w = L.chelis_tensor_write_view(g)
    arr = np.ctypeslib.as_array(ctypes.cast(w.data, ctypes.POINTER(ctypes.c_double)), (15,))
    arr[:] = np.arange(15)
    L.chelis_tensor_end_write(g)
    v = L.chelis_tensor_read_view(t)
    assert np.ctypeslib.as_array(ctypes.cast(v.data, ctypes.POINTER(ctypes.c_double)), (15,)).sum() == 105
    L.chelis_tensor_release(t)
    assert L.chelis_dtype_size(C.DT_F32) == 4 and L.chelis_dtype_size(C.DT_I64) == 8
    assert L.chelis_key_from_seed(-1) == 2**64 - 1


def test_metadata_plans():
    L = C.lib()
    arr = (C.Scalar * 3)(*[C.i64(v) for v in (2, 3, 4)])
    ex = C.Scalar()
    ex.dtype = C.DT_F32
    p = L.chelis_metadata_plan_new(C.i64(3), arr, ex)
    assert L.chelis_metadata_plan_count(p) == 24 and L.chelis_metadata_plan_byte_count(p) == 96
    assert [L.chelis_metadata_plan_strides(p)[i] for i in range(3)] == [12, 4, 1]
    assert L.chelis_metadata_plan_byte_offset(p, C.i64(23)) == 92
    L.chelis_metadata_plan_release(p)
    # a transposed view of a [3, 2] buffer
    sh = (C.Scalar * 2)(C.i64(2), C.i64(3))
    st = (C.Scalar * 2)(C.i64(1), C.i64(2))
    v = L.chelis_metadata_plan_view(C.i64(2), sh, st, ex, C.i64(24))
    assert [L.chelis_metadata_plan_byte_offset(v, C.i64(i)) for i in range(6)] == [0, 8, 16, 4, 12, 20]
    L.chelis_metadata_plan_release(v)


TRAP_CASES = {
    "negative_extent": "p = L.chelis_metadata_plan_new(C.i64(1), (C.Scalar * 1)(C.i64(-1)), ex)",
    "short_capacity": "p = L.chelis_metadata_plan_view(C.i64(1), (C.Scalar * 1)(C.i64(4)), (C.Scalar * 1)(C.i64(1)), ex, C.i64(15))",
    "negative_stride": "p = L.chelis_metadata_plan_view(C.i64(1), (C.Scalar * 1)(C.i64(4)), (C.Scalar * 1)(C.i64(-1)), ex, C.i64(64))",
    "overflow": "p = L.chelis_metadata_plan_new(C.i64(2), (C.Scalar * 2)(C.i64(2**62), C.i64(4)), ex)",
}


@pytest.mark.parametrize("case", sorted(TRAP_CASES))
def test_metadata_plan_traps_like_the_reference(case):
    """Invalid plans end the process with status 1 and the reference's trap
    text (crates/chelis-backend-hip/runtime/chelis_device_owner.cpp:14-20)."""
    code = textwrap.dedent(f"""
        import sys; sys.path.insert(0, {ROOT!r})
        import chelis_amd as C
        L = C.lib(); ex = C.Scalar(); ex.dtype = C.DT_F32
        {TRAP_CASES[case]}
        print("no trap")
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    kind = "overflow" if case == "overflow" else "domain"
    assert f"numeric trap: {kind} in metadata_plan at i64" in r.stderr


def _cut_closed_form(rate, f32):
    """The least m in [0, 2^53] whose unit m * 2^-53, taken to the dtype, is
    not below the dtype's rate, from exact rationals: binary64 compares the
    unit itself; binary32 rounds it to nearest even, so the unit is not below
    r exactly above the midpoint between r and its predecessor (at the
    midpoint when r's significand is even)."""
    from fractions import Fraction
    if not f32:
        q = Fraction(rate) * 2 ** 53
        return int(q) if q.denominator == 1 else int(q) + 1
    r = np.float32(rate)
    if r == 0:
        return 0
    p = np.nextafter(r, np.float32(0))
    mid = (Fraction(float(p)) + Fraction(float(r))) / 2 * 2 ** 53
    r_even = (int(r.view(np.uint32)) & 1) == 0
    if mid.denominator == 1:
        return int(mid) if r_even else int(mid) + 1
    return int(mid) + 1


@pytest.mark.parametrize("rate", [0.0, 0.1, 0.5, 0.25, 1e-30, 1e-45, 0.9999999, 0.3333333333333333,
                                  float(np.nextafter(np.float32(0.5), np.float32(1))),
                                  2.0 ** -53, 1 - 2.0 ** -53, 0.7])
@pytest.mark.parametrize("dtype", [0, 1])
def test_dropout_cut_is_the_drop_test(rate, dtype):
    """chelis_hip_dropout_cut, the integer form of [05-OP-37]'s unit < rate
    the dropout kernels run, against its closed form."""
    f32 = dtype == 0
    if f32 and float(np.float32(rate)) >= 1.0:
        pytest.skip("the binary32 rate rounds to 1")
    L = C.lib()
    L.chelis_hip_dropout_cut.restype = ctypes.c_uint64
    L.chelis_hip_dropout_cut.argtypes = [ctypes.c_double, ctypes.c_int32]
    assert L.chelis_hip_dropout_cut(rate, dtype) == _cut_closed_form(rate, f32)

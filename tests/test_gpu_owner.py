"""The device owner API on the GPU (include/chelis_device_owner.h; contract
crates/chelis-backend-hip/runtime/chelis_device_owner.h:16-24): import of a
foreign packet and a launcher over it, borrow, clone and copy_to_host of
strided, transposed and broadcast views against numpy's own indexing, and
the traps an invalid request ends in (run in child processes, since a trap
ends the process with status 1)."""
import ctypes
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import chelis_amd as C
from oracle import oracle as O

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TRAP = "numeric trap: domain in metadata_plan at i64"


def setup_module(_m):
    O.build()


def packet_of(t):
    return t.packet.contents


def test_import_packet_then_launch():
    """The reference loader's input path: a borrowed packet imported, its
    view handed to a launcher (softmax), the result bit-equal to the oracle."""
    x = (np.random.default_rng(1).standard_normal((64, 1024)) * 2).astype(np.float32)
    base = C.to_device(x)
    p = packet_of(base)
    owner = C.import_packet(x.shape, (1024, 1), p.data, p.byte_capacity, C.DT_F32)
    v = C.lib().chelis_device_tensor_view(owner).contents
    assert v.data == p.data and v.ownership == 0 and v.count == x.size and v.rank == 2
    assert v.byte_capacity == x.nbytes and (v.shape[0], v.shape[1]) == x.shape
    assert C.lib().chelis_device_tensor_device(owner) == 0
    y = C.empty(x.shape, np.float32)
    C.check(C.lib().chelis_hip_softmax(C.lib().chelis_device_tensor_view(owner), y.packet), "softmax")
    assert np.array_equal(y.numpy().view(np.uint32), O.softmax_rows(x).view(np.uint32))
    C.lib().chelis_device_tensor_release(owner)
    # the base storage is untouched by releasing the borrowed owner
    assert np.array_equal(base.numpy(), x)


def test_alloc_zero_fills_and_packet_fields():
    t = C.empty((3, 5, 7), np.float64)
    p = packet_of(t)
    assert p.ownership == 1 and p.count == 105 and p.byte_capacity == 105 * 8 and p.rank == 3
    assert [p.strides[i] for i in range(3)] == [35, 7, 1]
    assert np.array_equal(t.numpy(), np.zeros((3, 5, 7)))
    e = C.empty((4, 0), np.float32)
    assert packet_of(e).count == 0 and e.numpy().shape == (4, 0)


def test_borrow_shares_storage():
    x = np.arange(48, dtype=np.int64).reshape(6, 8)
    base = C.to_device(x)
    p = packet_of(base)
    b = C.borrow((8, 6), np.int64, p.data, p.byte_capacity)  # a reshape over the same bytes
    bp = packet_of(b)
    assert bp.ownership == 0 and bp.data == p.data
    assert np.array_equal(b.numpy(), x.reshape(8, 6))
    del b
    assert np.array_equal(base.numpy(), x)


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.uint8, np.int64, np.float16])
def test_clone_and_copy_to_host_of_strided_views(dtype):
    rng = np.random.default_rng(3)
    a = (rng.standard_normal((37, 53)) * 100).astype(dtype)
    base = C.to_device(a)
    # transposed
    t = base.view((53, 37), (1, 53))
    assert np.array_equal(t.numpy(), a.T)
    c = C.clone(t)
    assert packet_of(c).ownership == 1 and [packet_of(c).strides[i] for i in range(2)] == [37, 1]
    assert np.array_equal(c.numpy(), a.T)
    # broadcast of one row (stride 0) and of one column
    r = base.view((5, 53), (0, 1), 53 * 4)
    assert np.array_equal(C.clone(r).numpy(), np.broadcast_to(a[4], (5, 53)))
    col = base.view((37, 9), (53, 0), 2)
    assert np.array_equal(col.numpy(), np.broadcast_to(a[:, 2:3], (37, 9)))
    # every other row and column, from an offset
    s = base.view((18, 26), (106, 2), 1)
    assert np.array_equal(C.clone(s).numpy(), a[0:36:2, 1:53:2])
    # a dense view clones as one copy
    assert np.array_equal(C.clone(base).numpy(), a)


def test_clone_of_high_rank_views():
    """Views whose axes do not merge: rank 6 (one kernel launch) and rank 14
    with extent 2 on every axis (more axes than the copy kernel takes, so the
    host peels leading axes)."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal(2 ** 16).astype(np.float32)
    base = C.to_device(x)
    shape6, strides6 = (3, 4, 2, 5, 2, 3), (4000, 7, 600, 60, 3001, 2)
    ref6 = np.lib.stride_tricks.as_strided(x, shape6, [s * 4 for s in strides6])
    assert np.array_equal(C.clone(base.view(shape6, strides6)).numpy(), ref6)
    shape14 = (2,) * 14
    strides14 = tuple(2 ** (14 - i) + (i % 3) for i in range(14))
    span = sum((e - 1) * s for e, s in zip(shape14, strides14)) + 1
    assert span <= x.size
    ref14 = np.lib.stride_tricks.as_strided(x, shape14, [s * 4 for s in strides14])
    v = base.view(shape14, strides14)
    assert np.array_equal(C.clone(v).numpy(), ref14)
    assert np.array_equal(v.numpy(), ref14)


def _child(body: str):
    code = textwrap.dedent(f"""
        import sys, ctypes, numpy as np
        sys.path.insert(0, {ROOT!r})
        import chelis_amd as C
        L = C.lib()
    """) + textwrap.dedent(body)
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)


TRAP_CASES = {
    "import_null": "L.chelis_device_tensor_import(None)",
    "import_owned_packet": """
        t = C.empty((4,), np.float32); p = t.packet.contents
        g, keep = C.make_packet((4,), (1,), p.data, 16, C.DT_F32, ownership=1)
        L.chelis_device_tensor_import(ctypes.byref(g))
    """,
    "import_reserved_bytes": """
        t = C.empty((4,), np.float32); p = t.packet.contents
        g, keep = C.make_packet((4,), (1,), p.data, 16, C.DT_F32)
        g.reserved[1] = 7
        L.chelis_device_tensor_import(ctypes.byref(g))
    """,
    "import_past_capacity": """
        t = C.empty((4,), np.float32); p = t.packet.contents
        C.import_packet((4,), (2,), p.data, 16, C.DT_F32)
    """,
    "import_host_memory": """
        a = np.zeros(4, np.float32)
        C.import_packet((4,), (1,), a.ctypes.data, 16, C.DT_F32)
    """,
    "import_misaligned": """
        t = C.empty((8,), np.float32); p = t.packet.contents
        C.import_packet((2,), (1,), p.data + 2, 16, C.DT_F32)
    """,
    "import_count_mismatch": """
        t = C.empty((4,), np.float32); p = t.packet.contents
        g, keep = C.make_packet((4,), (1,), p.data, 16, C.DT_F32)
        g.count = 3
        L.chelis_device_tensor_import(ctypes.byref(g))
    """,
    "copy_from_host_into_borrowed": """
        t = C.empty((4,), np.float32); p = t.packet.contents
        b = C.borrow((4,), np.float32, p.data, 16)
        a = np.ones(4, np.float32)
        sh = (ctypes.c_int64 * 1)(4)
        h = L.chelis_tensor_entry_borrow(1, sh, C.DT_F32, a.ctypes.data, 16)
        L.chelis_device_tensor_copy_from_host(b.owner, h)
    """,
    "copy_to_host_count_mismatch": """
        t = C.empty((4,), np.float32)
        out = np.empty(5, np.float32)
        sh = (ctypes.c_int64 * 1)(5)
        h = L.chelis_tensor_entry_borrow(1, sh, C.DT_F32, out.ctypes.data, 20)
        g = L.chelis_tensor_begin_write(h)
        L.chelis_device_tensor_copy_to_host(g, t.owner)
    """,
    "view_of_null": "L.chelis_device_tensor_view(None)",
    "clone_of_null": "L.chelis_device_tensor_clone(None)",
    "release_of_null": "L.chelis_device_tensor_release(None)",
    "alloc_negative_extent": "C.empty((-1,), np.float32)",
}


@pytest.mark.parametrize("case", sorted(TRAP_CASES))
def test_invalid_requests_trap_domain(case):
    r = _child(TRAP_CASES[case])
    assert r.returncode == 1, (r.returncode, r.stderr[-2000:])
    assert TRAP in r.stderr, r.stderr[-2000:]


def test_a_valid_child_exits_zero():
    r = _child("""
        t = C.to_device(np.arange(6, dtype=np.float32))
        assert C.clone(t.view((3,), (2,))).numpy().tolist() == [0.0, 2.0, 4.0]
    """)
    assert r.returncode == 0, r.stderr[-2000:]

"""chelis_amd: MI355X-native execution of fused Chelis tensor regions.

The product is the C-ABI library ``libchelis_hip.so`` (headers in
``include/``). This module is the host-side Python mirror of the
reference's own binding flow (crates/chelis-python/src/native_tensor.rs:
210-240): it resolves the same owner symbols by name, moves numpy arrays
through ``chelis_device_tensor_alloc`` / ``copy_from_host`` /
``copy_to_host``, and calls the region launchers and program entries.

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import subprocess
import os
from ctypes import POINTER, c_double, c_int32, c_int64, c_uint8, c_uint64, c_void_p

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libchelis_hip.so")


class ChelisError(RuntimeError):
    pass


# ---- ABI types (include/chelis_runtime.h, include/chelis_device_descriptor.h) ----
DT_F32, DT_F64, DT_I32, DT_BOOL, DT_I64, DT_BF16, DT_F16, DT_I8, DT_I16, DT_KEY = 0, 1, 2, 3, 4, 5, 6, 7, 8, 9
# bfloat16 has no numpy dtype: bf16 tensors travel as np.uint16 bit patterns
_NP2DT = {np.dtype(np.float32): DT_F32, np.dtype(np.float64): DT_F64, np.dtype(np.int32): DT_I32,
          np.dtype(np.uint8): DT_BOOL, np.dtype(np.bool_): DT_BOOL, np.dtype(np.int64): DT_I64,
          np.dtype(np.uint16): DT_BF16, np.dtype(np.float16): DT_F16, np.dtype(np.int8): DT_I8,
          np.dtype(np.int16): DT_I16}
_DT2NP = {DT_F32: np.float32, DT_F64: np.float64, DT_I32: np.int32, DT_BOOL: np.uint8, DT_I64: np.int64,
          DT_BF16: np.uint16, DT_F16: np.float16, DT_I8: np.int8, DT_I16: np.int16, DT_KEY: np.uint64}


class Scalar(ctypes.Structure):
    _fields_ = [("dtype", c_uint8), ("reserved", c_uint8 * 7), ("bits", c_uint64)]


class ReadView(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("count", c_int64), ("dtype", c_uint8), ("reserved", c_uint8 * 7)]


class GpuTensor(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("shape", POINTER(c_int64)), ("strides", POINTER(c_int64)),
                ("count", c_int64), ("byte_capacity", c_int64), ("rank", c_int32), ("dtype", c_uint8),
                ("ownership", c_uint8), ("reserved", c_uint8 * 2)]


class NumericFailure(ctypes.Structure):
    _fields_ = [("index", c_int64), ("kind", c_int32), ("reserved", c_int32), ("message", ctypes.c_char * 96)]


class FusedStep(ctypes.Structure):
    _fields_ = [("op", c_uint8), ("reserved", c_uint8 * 3), ("args", c_int32 * 2), ("imm", c_double)]


class FusedChain(ctypes.Structure):
    _fields_ = [("n_steps", c_int32), ("reserved", c_int32), ("steps", FusedStep * 16)]


P = POINTER(GpuTensor)

# Every exported symbol the headers in include/ declare, with its ctypes
# signature (restype, argtypes). tests/test_abi.py checks the library
# exports exactly these names.
SIGNATURES = {
    # chelis_runtime.h
    "chelis_alloc": (c_void_p, [c_int32, POINTER(c_int64), c_uint8]),
    "chelis_tensor_entry_borrow": (c_void_p, [c_int32, POINTER(c_int64), c_uint8, c_void_p, c_int64]),
    "chelis_tensor_retain": (None, [c_void_p]),
    "chelis_tensor_release": (None, [c_void_p]),
    "chelis_tensor_read_view": (ReadView, [c_void_p]),
    "chelis_tensor_begin_write": (c_void_p, [c_void_p]),
    "chelis_tensor_write_view": (ReadView, [c_void_p]),
    "chelis_tensor_end_write": (None, [c_void_p]),
    "chelis_dtype_size": (c_int64, [c_uint8]),
    "chelis_scalar_from_bits": (Scalar, [c_uint8, c_uint64]),
    "chelis_key_from_seed": (c_uint64, [c_int64]),
    "chelis_tensor_rank": (c_int32, [c_void_p]),
    "chelis_tensor_shape": (c_int64, [c_void_p, c_int32]),
    "chelis_tensor_numel": (c_int64, [c_void_p]),
    "chelis_metadata_plan_new": (c_void_p, [Scalar, POINTER(Scalar), Scalar]),
    "chelis_metadata_plan_view": (c_void_p, [Scalar, POINTER(Scalar), POINTER(Scalar), Scalar, Scalar]),
    "chelis_metadata_plan_rank": (c_int32, [c_void_p]),
    "chelis_metadata_plan_shape": (POINTER(c_int64), [c_void_p]),
    "chelis_metadata_plan_strides": (POINTER(c_int64), [c_void_p]),
    "chelis_metadata_plan_count": (c_int64, [c_void_p]),
    "chelis_metadata_plan_byte_count": (c_int64, [c_void_p]),
    "chelis_metadata_plan_byte_offset": (c_int64, [c_void_p, Scalar]),
    "chelis_metadata_plan_dtype": (c_uint8, [c_void_p]),
    "chelis_metadata_plan_check_capacity": (None, [c_void_p, Scalar]),
    "chelis_metadata_plan_release": (None, [c_void_p]),
    "chelis_contiguous": (c_void_p, [c_void_p]),
    # chelis_device_owner.h
    "chelis_device_tensor_alloc": (c_void_p, [c_void_p]),
    "chelis_device_tensor_borrow": (c_void_p, [c_void_p, c_void_p, Scalar]),
    "chelis_device_tensor_import": (c_void_p, [P]),
    "chelis_device_tensor_view": (P, [c_void_p]),
    "chelis_device_tensor_device": (c_int32, [c_void_p]),
    "chelis_device_tensor_clone": (c_void_p, [c_void_p]),
    "chelis_device_tensor_release": (None, [c_void_p]),
    "chelis_device_tensor_copy_from_host": (None, [c_void_p, c_void_p]),
    "chelis_device_tensor_copy_to_host": (None, [c_void_p, c_void_p]),
    # chelis_hip.h
    "chelis_hip_last_error": (ctypes.c_char_p, []),
    "chelis_hip_stream": (c_void_p, []),
    "chelis_hip_synchronize": (c_int32, []),
    "chelis_hip_build_info": (ctypes.c_char_p, []),
    "chelis_hip_softmax": (c_int32, [P, P]),
    "chelis_hip_scaled_masked_softmax": (c_int32, [P, c_double, c_int32, P]),
    "chelis_hip_causal_attention": (c_int32, [P, P, P, c_double, P]),
    "chelis_hip_softmax_adjoint": (c_int32, [P, P, P]),
    "chelis_hip_layer_norm": (c_int32, [P, P, P, c_double, P]),
    "chelis_hip_fused_elementwise": (c_int32, [POINTER(FusedChain), POINTER(P), c_int32, P]),
    "chelis_hip_gelu": (c_int32, [P, P]),
    "chelis_hip_relu": (c_int32, [P, P]),
    "chelis_hip_relu_adjoint": (c_int32, [P, P, P]),
    "chelis_hip_dropout": (c_int32, [c_uint64, P, c_double, P]),
    "chelis_hip_dropout_replay": (c_int32, [c_uint64, P, c_double, P]),
    "chelis_hip_uniform_like": (c_int32, [c_uint64, c_double, c_double, P]),
    "chelis_hip_reduce": (c_int32, [c_int32, POINTER(FusedChain), POINTER(P), c_int32, c_int32, P]),
    "chelis_hip_reduce_static": (c_int32, [c_int32, POINTER(FusedChain), POINTER(P), c_int32, c_int32, P]),
    "chelis_hip_count": (c_int32, [P, c_int32, P, POINTER(c_int32)]),
    "chelis_hip_trap_status": (c_int32, [POINTER(c_int32)]),
    "chelis_hip_matmul": (c_int32, [P, P, P, c_int32]),
    "chelis_hip_linear": (c_int32, [P, P, P, c_int32, P, P, c_int32]),
    # chelis_programs.h
    "chelis_prog_linreg_step": (c_int32, [POINTER(P), c_int32, POINTER(P), c_int32]),
    "chelis_prog_transformer_block": (c_int32, [POINTER(P), c_int32, POINTER(P), c_int32]),
    "chelis_prog_mlp_train_step": (c_int32, [POINTER(P), c_int32, POINTER(P), c_int32]),
    "linreg_step_device": (None, [POINTER(c_void_p), c_int32, POINTER(c_void_p), c_int32]),
    "transformer_block_device": (None, [POINTER(c_void_p), c_int32, POINTER(c_void_p), c_int32]),
    "mlp_train_step_device": (None, [POINTER(c_void_p), c_int32, POINTER(c_void_p), c_int32]),
    "chelis_hip_compare": (c_int32, [c_int32, P, P, P]),
    "chelis_hip_logical": (c_int32, [c_int32, P, P, P]),
    "chelis_hip_where": (c_int32, [P, P, P, P]),
    "chelis_hip_extrema_adjoint": (c_int32, [c_int32, c_int32, P, P, P, P]),
    "chelis_hip_cast": (c_int32, [P, P, POINTER(NumericFailure)]),
    "chelis_hip_integer_elementwise": (c_int32, [c_int32, P, P, P, POINTER(NumericFailure)]),
    "chelis_hip_gather": (c_int32, [P, P, c_int32, c_int32, P, POINTER(NumericFailure)]),
    "chelis_hip_take_numeric_failure": (c_int32, [POINTER(NumericFailure)]),
    "chelis_hip_cumsum": (c_int32, [P, c_int32, c_int32, P, POINTER(NumericFailure)]),
    "chelis_hip_pad": (c_int32, [P, POINTER(c_int64), ctypes.c_uint64, P]),
    "chelis_hip_scatter": (c_int32, [c_int32, P, P, P, c_int32, c_int32, P, POINTER(NumericFailure)]),
    "chelis_hip_scatter_elements": (c_int32, [P, P, P, c_int32, P, POINTER(NumericFailure)]),
    "chelis_hip_allocation_counts": (None, [POINTER(c_int64), POINTER(c_int64)]),
    "chelis_hip_set_exact_matmul": (c_int32, [c_int32]),
    "chelis_hip_set_exact": (c_int32, [c_int32]),
    # chelis_dag.h
    "chelis_dag_compile": (c_void_p, [ctypes.c_char_p, c_int64]),
    "chelis_dag_release": (None, [c_void_p]),
    "chelis_dag_run": (c_int32, [c_void_p, POINTER(P), c_int32, POINTER(P), c_int32]),
    "chelis_dag_input_count": (c_int32, [c_void_p]),
    "chelis_dag_output_count": (c_int32, [c_void_p]),
    "chelis_dag_label": (ctypes.c_char_p, [c_void_p, c_int32, c_int32]),
    "chelis_dag_type": (c_int32, [c_void_p, c_int32, c_int32, POINTER(c_int32), POINTER(c_int64), c_int32,
                                  POINTER(c_int32)]),
    "chelis_dag_peak_device_bytes": (c_int64, [c_void_p]),
    "chelis_dag_peak_device_bytes_at": (c_int64, [c_void_p, POINTER(c_int64), c_int32]),
    "chelis_dag_symbol_count": (c_int32, [c_void_p]),
    "chelis_dag_symbol_name": (ctypes.c_char_p, [c_void_p, c_int32]),
    "chelis_dag_output_shape": (c_int32, [c_void_p, POINTER(P), c_int32, c_int32, POINTER(c_int32),
                                          POINTER(c_int64), c_int32]),
    "chelis_dag_launch_count": (c_int64, [c_void_p]),
    "chelis_dag_describe": (ctypes.c_char_p, [c_void_p]),
    "chelis_dag_fuse": (ctypes.c_char_p, [ctypes.c_char_p, c_int64]),
    "chelis_codegen_hip": (c_void_p, [ctypes.c_char_p, c_int64, ctypes.c_char_p]),
    "chelis_prepare_dag_for_codegen": (ctypes.c_char_p, [ctypes.c_char_p, c_int64]),
    "chelis_hip_tensor_capable_prims": (c_int32, [POINTER(POINTER(c_uint8))]),
    "chelis_hip_runtime_dir": (ctypes.c_char_p, []),
    "chelis_codegen_hip_host_program": (c_void_p, [c_int32, POINTER(ctypes.c_char_p), POINTER(ctypes.c_char_p),
                                                   POINTER(c_int64)]),
    "chelis_host_program_release": (None, [c_void_p]),
    "chelis_host_program_helper_count": (c_int32, [c_void_p]),
    "chelis_host_program_helper_name": (ctypes.c_char_p, [c_void_p, c_int32]),
    "chelis_host_program_helper": (c_void_p, [c_void_p, c_int32]),
    "chelis_codegen_release": (None, [c_void_p]),
    "chelis_codegen_c_source": (ctypes.c_char_p, [c_void_p]),
    "chelis_codegen_h_header": (ctypes.c_char_p, [c_void_p]),
    "chelis_codegen_list_count": (c_int32, [c_void_p, c_int32]),
    "chelis_codegen_list_item": (ctypes.c_char_p, [c_void_p, c_int32, c_int32]),
    "chelis_codegen_peak_device_bytes_formula": (ctypes.c_char_p, [c_void_p]),
    "chelis_codegen_peak_device_bytes_estimate": (c_int64, [c_void_p]),
    "linreg_step": (None, [POINTER(c_void_p), ctypes.c_int, POINTER(c_void_p), ctypes.c_int]),
    "transformer_block": (None, [POINTER(c_void_p), ctypes.c_int, POINTER(c_void_p), ctypes.c_int]),
    "mlp_train_step": (None, [POINTER(c_void_p), ctypes.c_int, POINTER(c_void_p), ctypes.c_int]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The product library. Raises if it was not built: no fallback exists."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ChelisError(f"{LIB_PATH} is missing: build it with `python -m chelis_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = lib().chelis_hip_last_error().decode(errors="replace")
        raise ChelisError(f"{what or 'chelis_hip'} failed (status {status}): {msg}")


def synchronize() -> None:
    check(lib().chelis_hip_synchronize(), "synchronize")


def i64(v: int) -> Scalar:
    return lib().chelis_scalar_from_bits(DT_I64, int(v) & (2**64 - 1))


# ---- device tensors through the owner API ----
class DeviceTensor:
    """An owned (or borrowed) device tensor: a chelis_device_tensor_owner."""

    def __init__(self, owner: int, keep=None):
        self.owner = owner
        self._keep = keep
        self.packet = lib().chelis_device_tensor_view(owner)
        p = self.packet.contents
        self.shape = tuple(p.shape[i] for i in range(p.rank))
        self.strides = tuple(p.strides[i] for i in range(p.rank))
        self.dtype = np.dtype(_DT2NP[p.dtype])
        self.data = p.data

    def __del__(self):
        try:
            if self.owner:
                lib().chelis_device_tensor_release(self.owner)
                self.owner = None
        except Exception:
            pass

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def view(self, shape, strides, offset_elems: int = 0) -> "View":
        """A strided packet over this tensor's storage (a transposed or
        broadcast operand), borrowed for as long as the View lives."""
        return View(self, shape, strides, offset_elems)

    def numpy(self) -> np.ndarray:
        return to_host(self)


class View:
    """A strided view of a device tensor's storage, made the way the
    reference's Python loader hands a foreign tensor to a compiled entry
    (crates/chelis-python/src/native_tensor.rs:210-240): a borrowed packet
    imported through chelis_device_tensor_import. The view's owner borrows
    the base storage and is released with the View."""

    def __init__(self, base: DeviceTensor, shape, strides, offset: int = 0):
        self.base = base
        self.shape = tuple(int(s) for s in shape)
        self.strides = tuple(int(s) for s in strides)
        self.dtype = base.dtype
        bp = base.packet.contents
        self.owner = import_packet(self.shape, self.strides, (bp.data or 0) + offset * self.dtype.itemsize,
                                   bp.byte_capacity - offset * self.dtype.itemsize, bp.dtype)
        self.packet = lib().chelis_device_tensor_view(self.owner)

    def numpy(self) -> np.ndarray:
        return to_host(self)

    def __del__(self):
        try:
            if self.owner:
                lib().chelis_device_tensor_release(self.owner)
                self.owner = None
        except Exception:
            pass


def make_packet(shape, strides, data: int, byte_capacity: int, dtype_tag: int, ownership: int = 0):
    """A chelis_gpu_tensor over caller memory; returns (packet, keep-alive)."""
    shape = tuple(int(s) for s in shape)
    sh = (c_int64 * max(1, len(shape)))(*shape)
    st = (c_int64 * max(1, len(strides)))(*[int(s) for s in strides])
    g = GpuTensor()
    g.data = data or None
    g.shape = ctypes.cast(sh, POINTER(c_int64))
    g.strides = ctypes.cast(st, POINTER(c_int64))
    g.count = int(np.prod(shape, dtype=np.int64))
    g.byte_capacity = int(byte_capacity)
    g.rank = len(shape)
    g.dtype = dtype_tag
    g.ownership = ownership
    return g, (sh, st)


def import_packet(shape, strides, data: int, byte_capacity: int, dtype_tag: int) -> int:
    """chelis_device_tensor_import of a borrowed packet: a new owner handle."""
    g, keep = make_packet(shape, strides, data, byte_capacity, dtype_tag)
    owner = lib().chelis_device_tensor_import(ctypes.byref(g))
    del keep
    return owner


def borrow(shape, dtype, data: int, byte_capacity: int) -> "DeviceTensor":
    """chelis_device_tensor_borrow: a row-major owner over caller storage."""
    return DeviceTensor(lib().chelis_device_tensor_borrow(_plan(shape, dtype), data, i64(byte_capacity)))


def clone(t) -> "DeviceTensor":
    """chelis_device_tensor_clone: an owned dense copy of a tensor or view."""
    return DeviceTensor(lib().chelis_device_tensor_clone(t.owner))


def _plan(shape, dtype, tag=None) -> int:
    shape = tuple(int(s) for s in shape)
    arr = (Scalar * max(1, len(shape)))(*[i64(s) for s in shape])
    ex = Scalar()
    ex.dtype = _NP2DT[np.dtype(dtype)] if tag is None else tag
    return lib().chelis_metadata_plan_new(i64(len(shape)), arr, ex)


def empty(shape, dtype) -> DeviceTensor:
    """chelis_device_tensor_alloc: a zero-filled owned device tensor."""
    return DeviceTensor(lib().chelis_device_tensor_alloc(_plan(shape, dtype)))


def to_device(a: np.ndarray) -> DeviceTensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.bool_:
        a = a.view(np.uint8)
    t = empty(a.shape, a.dtype)
    shape = (c_int64 * max(1, a.ndim))(*a.shape)
    host = lib().chelis_tensor_entry_borrow(a.ndim, shape, _NP2DT[a.dtype], a.ctypes.data, a.nbytes)
    lib().chelis_device_tensor_copy_from_host(t.owner, host)
    lib().chelis_tensor_release(host)
    return t


def to_host(t) -> np.ndarray:
    """chelis_device_tensor_copy_to_host of a DeviceTensor or a View (a
    strided view is gathered on the device first) into a fresh array."""
    out = np.empty(t.shape, t.dtype)
    shape = (c_int64 * max(1, out.ndim))(*out.shape)
    host = lib().chelis_tensor_entry_borrow(out.ndim, shape, _NP2DT[out.dtype], out.ctypes.data, out.nbytes)
    guard = lib().chelis_tensor_begin_write(host)
    lib().chelis_device_tensor_copy_to_host(guard, t.owner)
    lib().chelis_tensor_end_write(guard)
    lib().chelis_tensor_release(host)
    return out


def _p(t):
    return t.packet


# ---- region launchers (asynchronous on the library stream) ----
def softmax(x, y=None):
    y = y or empty(x.shape, x.dtype)
    check(lib().chelis_hip_softmax(_p(x), _p(y)), "softmax")
    return y


def scaled_masked_softmax(x, scale: float, causal: bool, y=None):
    y = y or empty(x.shape, x.dtype)
    check(lib().chelis_hip_scaled_masked_softmax(_p(x), scale, int(causal), _p(y)), "scaled_masked_softmax")
    return y


def causal_attention(q, k, v, scale: float, o=None):
    """softmax(where(key <= row, q.k^T * scale, -inf)).v in one launch over
    f32 [batch, heads, seq, 64] views."""
    o = o or empty(q.shape, q.dtype)
    check(lib().chelis_hip_causal_attention(_p(q), _p(k), _p(v), scale, _p(o)), "causal_attention")
    return o


def softmax_adjoint(y, g, dx=None):
    dx = dx or empty(y.shape, y.dtype)
    check(lib().chelis_hip_softmax_adjoint(_p(y), _p(g), _p(dx)), "softmax_adjoint")
    return dx


def layer_norm(x, gamma, beta, eps: float, y=None):
    y = y or empty(x.shape, x.dtype)
    check(lib().chelis_hip_layer_norm(_p(x), _p(gamma), _p(beta), eps, _p(y)), "layer_norm")
    return y


def gelu(x, y=None):
    y = y or empty(x.shape, x.dtype)
    check(lib().chelis_hip_gelu(_p(x), _p(y)), "gelu")
    return y


def relu(x, y=None):
    y = y or empty(x.shape, x.dtype)
    check(lib().chelis_hip_relu(_p(x), _p(y)), "relu")
    return y


def relu_adjoint(x, g, dx=None):
    dx = dx or empty(x.shape, x.dtype)
    check(lib().chelis_hip_relu_adjoint(_p(x), _p(g), _p(dx)), "relu_adjoint")
    return dx


def dropout(key: int, x, rate: float, y=None):
    y = y or empty(x.shape, x.dtype)
    check(lib().chelis_hip_dropout(key & (2**64 - 1), _p(x), rate, _p(y)), "dropout")
    return y


def dropout_replay(key: int, g, rate: float, dx=None):
    dx = dx or empty(g.shape, g.dtype)
    check(lib().chelis_hip_dropout_replay(key & (2**64 - 1), _p(g), rate, _p(dx)), "dropout_replay")
    return dx


def uniform_like(key: int, low: float, high: float, out):
    check(lib().chelis_hip_uniform_like(key & (2**64 - 1), low, high, _p(out)), "uniform_like")
    return out


FUSED_OPS = ["add", "sub", "mul", "div", "max_elem", "min_elem", "neg", "recip", "exp", "log", "sqrt", "tanh",
             "erfc", "abs", "floor", "ceil", "round", "relu", "relu_adjoint", "const"]


def fused_chain(steps) -> FusedChain:
    """steps: list of (op_name, arg0, arg1[, imm]); args >= 0 index inputs,
    ('s', k) refers to step k."""
    ch = FusedChain()
    ch.n_steps = len(steps)
    for i, st in enumerate(steps):
        op, args = st[0], list(st[1:3]) + [0] * (2 - len(st[1:3]))
        ch.steps[i].op = FUSED_OPS.index(op)
        for j, a in enumerate(args[:2]):
            ch.steps[i].args[j] = -(a[1] + 1) if isinstance(a, tuple) else int(a)
        ch.steps[i].imm = float(st[3]) if len(st) > 3 else 0.0
    return ch


def fused_elementwise(chain: FusedChain, inputs, out):
    arr = (P * max(1, len(inputs)))(*[_p(t) for t in inputs])
    check(lib().chelis_hip_fused_elementwise(ctypes.byref(chain), arr, len(inputs), _p(out)), "fused_elementwise")
    return out


# ---- reductions ----
REDUCE_OPS = {"sum": 0, "max": 2, "min": 3, "prod": 4, "argmax": 5, "argmin": 6}


def reduce(op: str, inputs, axis: int, out=None, chain: FusedChain | None = None, static: bool = False):
    """chelis_hip_reduce over one axis; `chain` (with several inputs) is the
    inlined FusedElem leaf, else inputs is one tensor. static=True calls the
    allocation-free chelis_hip_reduce_static."""
    if not isinstance(inputs, (list, tuple)):
        inputs = [inputs]
    x0 = inputs[0]
    ax = axis % len(x0.shape)
    shape = x0.shape[:ax] + x0.shape[ax + 1:]
    if out is None:
        out = empty(shape, np.int64 if op in ("argmax", "argmin") else x0.dtype)
    arr = (P * len(inputs))(*[_p(t) for t in inputs])
    fn = lib().chelis_hip_reduce_static if static else lib().chelis_hip_reduce
    check(fn(REDUCE_OPS[op], ctypes.byref(chain) if chain is not None else None, arr, len(inputs), axis, _p(out)),
          f"reduce {op}")
    return out


def count(x, axis: int, out=None, deferred: bool = False):
    """chelis_hip_count: Bool8 -> i64; returns (out, error_code). With
    deferred=True the call does not wait and the code goes to the trap
    channel (trap_status); error_code is then None."""
    ax = axis % len(x.shape)
    if out is None:
        out = empty(x.shape[:ax] + x.shape[ax + 1:], np.int64)
    if deferred:
        check(lib().chelis_hip_count(_p(x), axis, _p(out), None), "count")
        return out, None
    err = c_int32(0)
    check(lib().chelis_hip_count(_p(x), axis, _p(out), ctypes.byref(err)), "count")
    return out, err.value


def trap_status() -> int:
    """chelis_hip_trap_status: waits for the library stream, returns and
    clears the codes deferred launches recorded (0: none)."""
    code = c_int32(0)
    check(lib().chelis_hip_trap_status(ctypes.byref(code)), "trap status")
    return code.value


# ---- comparison, logical, where, checked casts / integer arithmetic, gather ----
COMPARE_KINDS = {"cmp_lt": 0, "lt": 1, "eq": 2, "neq": 3, "gt": 4, "gte": 5, "lte": 6}
LOGICAL_KINDS = {"and": 0, "or": 1, "not": 2}
INT_OPS = {"add": 0, "sub": 1, "mul": 2, "floor_div": 3, "trunc_div": 4, "mod": 5, "max_elem": 6, "min_elem": 7,
           "neg": 8, "abs": 9, "bitand": 10, "bitor": 11, "bitxor": 12, "shl": 13, "shr": 14}


def _bshape(*ts):
    return tuple(np.broadcast_shapes(*[t.shape for t in ts]))


def _failure(f: NumericFailure):
    """(index, kind, trap line) of a failure record, None when it holds none."""
    return None if f.kind == 0 else (f.index, f.kind, f.message.decode())


def compare(kind: str, a, b, out=None):
    """chelis_hip_compare: Bool8 (np.uint8) result; operands of one rank
    broadcast by their extent-1 axes."""
    out = out or empty(_bshape(a, b), np.uint8)
    check(lib().chelis_hip_compare(COMPARE_KINDS[kind], _p(a), _p(b), _p(out)), "compare")
    return out


def logical(kind: str, a, b=None, out=None):
    out = out or empty(_bshape(a, b) if b is not None else a.shape, np.uint8)
    check(lib().chelis_hip_logical(LOGICAL_KINDS[kind], _p(a), _p(b) if b is not None else None, _p(out)),
          "logical")
    return out


def where(cond, a, b, out=None):
    out = out or empty(_bshape(cond, a, b), a.dtype)
    check(lib().chelis_hip_where(_p(cond), _p(a), _p(b), _p(out)), "where")
    return out


def extrema_adjoint(kind: str, operand: str, a, b, g, out=None):
    """chelis_hip_extrema_adjoint: kind "max" / "min", operand "left" / "right"."""
    out = out or empty(_bshape(a, b, g), g.dtype)
    check(lib().chelis_hip_extrema_adjoint(("max", "min").index(kind), ("left", "right").index(operand), _p(a),
                                           _p(b), _p(g), _p(out)), "extrema_adjoint")
    return out


def cast(x, dtype, out=None, deferred: bool = False):
    """chelis_hip_cast to `dtype` (np.uint16 for bf16, np.float16 for f16,
    np.uint8 for bool); returns (out, failure) with failure None when no
    element failed (and always None with deferred=True: the record goes to
    take_numeric_failure)."""
    out = out or empty(x.shape, dtype)
    f = NumericFailure()
    check(lib().chelis_hip_cast(_p(x), _p(out), None if deferred else ctypes.byref(f)), "cast")
    return out, None if deferred else _failure(f)


def integer_op(op: str, a, b=None, out=None, deferred: bool = False):
    """chelis_hip_integer_elementwise; returns (out, failure) as cast does."""
    out = out or empty(_bshape(a, b) if b is not None else a.shape, a.dtype)
    f = NumericFailure()
    check(lib().chelis_hip_integer_elementwise(INT_OPS[op], _p(a), _p(b) if b is not None else None, _p(out),
                                               None if deferred else ctypes.byref(f)), "integer_elementwise")
    return out, None if deferred else _failure(f)


def gather(values, indices, axis: int, batch_rank: int = 0, out=None, deferred: bool = False):
    """chelis_hip_gather; returns (out, failure) as cast does."""
    shape = tuple(values.shape[:axis]) + tuple(indices.shape[batch_rank:]) + tuple(values.shape[axis + 1:])
    out = out or empty(shape, values.dtype)
    f = NumericFailure()
    check(lib().chelis_hip_gather(_p(values), _p(indices), axis, batch_rank, _p(out),
                                  None if deferred else ctypes.byref(f)), "gather")
    return out, None if deferred else _failure(f)


def allocation_counts():
    """(scratch requests, device allocations) the library has made so far."""
    a, b = c_int64(0), c_int64(0)
    lib().chelis_hip_allocation_counts(ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value


def cumsum(x, axis: int, reverse: bool = False, out=None, deferred: bool = False):
    """chelis_hip_cumsum; returns (out, failure) as cast does. i8 / i16 scan
    into i32."""
    ax = axis % len(x.shape)
    if out is None:
        out = empty(x.shape, np.int32 if x.dtype in (np.int8, np.int16) else x.dtype)
    f = NumericFailure()
    check(lib().chelis_hip_cumsum(_p(x), ax, int(reverse), _p(out), None if deferred else ctypes.byref(f)), "cumsum")
    return out, None if deferred else _failure(f)


def pad(x, lo, hi, fill, out=None):
    """chelis_hip_pad: lo / hi elements before / after each axis; `fill` a
    value of x's dtype (bf16 as its 16-bit pattern)."""
    lo, hi = [int(v) for v in lo], [int(v) for v in hi]
    shape = tuple(int(e) + a + b for e, a, b in zip(x.shape, lo, hi))
    out = out or empty(shape, x.dtype)
    carrier = np.uint16 if x.dtype == np.uint16 else x.dtype
    bits = np.array([fill], carrier).view(np.dtype("u%d" % np.dtype(carrier).itemsize))[0]
    arr = (ctypes.c_int64 * max(1, len(lo)))(*lo)
    check(lib().chelis_hip_pad(_p(x), arr, int(bits), _p(out)), "pad")
    return out


def scatter(target, indices, updates, axis: int, batch_rank: int = 0, add: bool = False, out=None,
            deferred: bool = False):
    """chelis_hip_scatter (ScatterAdd when `add`, else the replacing
    Scatter); returns (out, failure) as cast does."""
    out = out or empty(target.shape, target.dtype)
    f = NumericFailure()
    check(lib().chelis_hip_scatter(int(add), _p(target), _p(indices), _p(updates), axis, batch_rank, _p(out),
                                   None if deferred else ctypes.byref(f)), "scatter")
    return out, None if deferred else _failure(f)


def scatter_elements(data, indices, updates, axis: int, out=None, deferred: bool = False):
    """chelis_hip_scatter_elements; returns (out, failure) as cast does."""
    out = out or empty(data.shape, data.dtype)
    f = NumericFailure()
    check(lib().chelis_hip_scatter_elements(_p(data), _p(indices), _p(updates), axis, _p(out),
                                            None if deferred else ctypes.byref(f)), "scatter_elements")
    return out, None if deferred else _failure(f)


def take_numeric_failure():
    """chelis_hip_take_numeric_failure: the earliest deferred failure since
    the last read as (index, kind, trap line), or None; clears the record."""
    f = NumericFailure()
    check(lib().chelis_hip_take_numeric_failure(ctypes.byref(f)), "take_numeric_failure")
    return _failure(f)


# ---- matmul ----
MATMUL_EXACT = 1
ACT = {None: 0, "none": 0, "relu": 1, "gelu": 2}


def _mm_shape(a, b):
    lead_a, lead_b = a.shape[:-2], b.shape[:-2]
    batch = tuple(np.broadcast_shapes(lead_a, lead_b)) if (lead_a or lead_b) else ()
    m = (a.shape[-2],) if len(a.shape) > 1 else ()
    n = (b.shape[-1],) if len(b.shape) > 1 else ()
    return batch + m + n


def matmul(a, b, c=None, exact: bool = False):
    if c is None:
        c = empty(_mm_shape(a, b), a.dtype)
    check(lib().chelis_hip_matmul(_p(a), _p(b), _p(c), MATMUL_EXACT if exact else 0), "matmul")
    return c


def linear(a, b, bias=None, act=None, residual=None, c=None, exact: bool = False):
    """c = act(a @ b + bias) + residual, fused in the matmul epilogue."""
    if c is None:
        c = empty(_mm_shape(a, b), a.dtype)
    check(lib().chelis_hip_linear(_p(a), _p(b), _p(bias) if bias is not None else None, ACT[act],
                                  _p(residual) if residual is not None else None, _p(c),
                                  MATMUL_EXACT if exact else 0), "linear")
    return c


def key_tensor(key: int) -> DeviceTensor:
    """A rank-0 KEY device tensor holding `key` (the RandomKey bits)."""
    t = DeviceTensor(lib().chelis_device_tensor_alloc(_plan((), np.uint64, DT_KEY)))
    host = np.array(key & (2**64 - 1), np.uint64)
    h = lib().chelis_tensor_entry_borrow(0, None, DT_KEY, host.ctypes.data, 8)
    lib().chelis_device_tensor_copy_from_host(t.owner, h)
    lib().chelis_tensor_release(h)
    return t


# ---- program entries (include/chelis_programs.h) ----
def program(name: str, inputs, outputs):
    """chelis_prog_{name}: enqueue the whole program; outputs are caller-owned."""
    ins = (P * len(inputs))(*[_p(t) for t in inputs])
    outs = (P * len(outputs))(*[_p(t) for t in outputs])
    check(getattr(lib(), f"chelis_prog_{name}")(ins, len(inputs), outs, len(outputs)), name)
    return outputs


def device_entry(name: str, inputs, n_out: int, library=None):
    """{name}_device: the reference's generated-entry ABI; returns owned
    outputs. `library` is the ctypes library defining it (this one by
    default)."""
    ins = (c_void_p * max(1, len(inputs)))(*[t.owner for t in inputs])
    outs = (c_void_p * max(1, n_out))()
    getattr(library or lib(), f"{name}_device")(ins, len(inputs), outs, n_out)
    return [DeviceTensor(outs[k]) for k in range(n_out)]


def host_entry(name: str, arrays, n_out: int, library=None):
    """{name}(chelis_tensor **, int, chelis_tensor **, int): the reference's
    host-tensor entry. numpy arrays in (borrowed as host tensors; a KEY input
    is passed as ("key", bits)), numpy arrays out (copied from the returned
    host tensors, which are then released)."""
    keep, hosts = [], []
    for a in arrays:
        if isinstance(a, tuple) and a[0] == "key":
            arr, tag = np.array(a[1] & (2**64 - 1), np.uint64), DT_KEY
        else:
            arr = np.ascontiguousarray(a)
            arr, tag = (arr.view(np.uint8), DT_BOOL) if arr.dtype == np.bool_ else (arr, _NP2DT[arr.dtype])
        shape = (c_int64 * max(1, arr.ndim))(*arr.shape)
        keep.append((arr, shape))
        hosts.append(lib().chelis_tensor_entry_borrow(arr.ndim, shape, tag, arr.ctypes.data, arr.nbytes))
    ins = (c_void_p * max(1, len(hosts)))(*hosts)
    outs = (c_void_p * max(1, n_out))()
    getattr(library or lib(), name)(ins, len(hosts), outs, n_out)
    result = []
    for o in outs[:n_out]:
        rank = lib().chelis_tensor_rank(o)
        shape = tuple(lib().chelis_tensor_shape(o, a) for a in range(rank))
        v = lib().chelis_tensor_read_view(o)
        dt = np.dtype(_DT2NP[v.dtype])
        result.append(np.ctypeslib.as_array(ctypes.cast(v.data, POINTER(ctypes.c_uint8)), (v.count * dt.itemsize,))
                      .view(dt).reshape(shape).copy() if v.count else np.zeros(shape, dt))
        lib().chelis_tensor_release(o)
    for h in hosts:
        lib().chelis_tensor_release(h)
    return result


def set_exact(on: bool) -> bool:
    """The library-wide exact mode (chelis_hip_set_exact): matmuls on the
    canonical-tree kernels and binary64 softmax rows with the correctly
    rounded exp, bit-identical to the C lane. Returns the previous mode."""
    return bool(lib().chelis_hip_set_exact(1 if on else 0))


def set_exact_matmul(on: bool) -> bool:
    """The same switch under its first name (chelis_hip_set_exact_matmul)."""
    return bool(lib().chelis_hip_set_exact_matmul(1 if on else 0))


# ---- the DAG front end (include/chelis_dag.h) ----
class DagProgram:
    """chelis_dag_compile / chelis_dag_run over a serde-form Chelis DAG."""

    def __init__(self, json_text: str):
        data = json_text.encode()
        self.handle = lib().chelis_dag_compile(data, len(data))
        if not self.handle:
            raise ChelisError("dag compile failed: " + lib().chelis_hip_last_error().decode(errors="replace"))
        kinds = [line.split()[1] for line in self.describe().splitlines() if len(line.split()) > 1]
        self.has_count = "count" in kinds
        # launches that record into the deferred failure record
        self.has_traps = any(k in ("cast", "integer", "gather", "cumsum", "scatter") for k in kinds)

    def __del__(self):
        try:
            if self.handle:
                lib().chelis_dag_release(self.handle)
                self.handle = None
        except Exception:
            pass

    def _slot(self, output: int, i: int):
        rank, dt = c_int32(), c_int32()
        shape = (c_int64 * 16)()
        check(lib().chelis_dag_type(self.handle, output, i, ctypes.byref(rank), shape, 16, ctypes.byref(dt)), "dag type")
        return tuple(shape[k] for k in range(rank.value)), dt.value

    @property
    def inputs(self):
        n = lib().chelis_dag_input_count(self.handle)
        return [(lib().chelis_dag_label(self.handle, 0, i).decode(),) + self._slot(0, i) for i in range(n)]

    @property
    def outputs(self):
        n = lib().chelis_dag_output_count(self.handle)
        return [(lib().chelis_dag_label(self.handle, 1, i).decode(),) + self._slot(1, i) for i in range(n)]

    def describe(self) -> str:
        return lib().chelis_dag_describe(self.handle).decode()

    @property
    def launches(self) -> int:
        return lib().chelis_dag_launch_count(self.handle)

    @property
    def peak_device_bytes(self) -> int:
        """Bytes one run needs; -1 when a run-time extent sizes them."""
        return lib().chelis_dag_peak_device_bytes(self.handle)

    @property
    def symbolic_dims(self):
        """The run-time extents, in binding order."""
        L = lib()
        return [L.chelis_dag_symbol_name(self.handle, k).decode() for k in range(L.chelis_dag_symbol_count(self.handle))]

    def peak_device_bytes_at(self, **extents) -> int:
        names = self.symbolic_dims
        vals = (c_int64 * max(1, len(names)))(*[int(extents[n]) for n in names])
        v = lib().chelis_dag_peak_device_bytes_at(self.handle, vals, len(names))
        if v < 0:
            raise ChelisError(lib().chelis_hip_last_error().decode(errors="replace"))
        return v

    def output_shapes(self, inputs):
        """Each output's shape for these inputs (run-time extents bound)."""
        ins = (P * max(1, len(inputs)))(*[_p(t) for t in inputs])
        shapes = []
        for o in range(lib().chelis_dag_output_count(self.handle)):
            rank = c_int32()
            shape = (c_int64 * 16)()
            check(lib().chelis_dag_output_shape(self.handle, ins, len(inputs), o, ctypes.byref(rank), shape, 16),
                  "dag output shape")
            shapes.append(tuple(shape[k] for k in range(rank.value)))
        return shapes

    def empty_outputs(self, inputs=None):
        if inputs is None:
            return [DeviceTensor(lib().chelis_device_tensor_alloc(_plan(shape, None, dt)))
                    for _, shape, dt in self.outputs]
        return [DeviceTensor(lib().chelis_device_tensor_alloc(_plan(shape, None, dt)))
                for shape, (_, _, dt) in zip(self.output_shapes(inputs), self.outputs)]

    def run(self, inputs, outputs=None):
        """Enqueue on the library stream; returns the output tensors."""
        outputs = outputs if outputs is not None else self.empty_outputs(inputs)
        ins = (P * max(1, len(inputs)))(*[_p(t) for t in inputs])
        outs = (P * max(1, len(outputs)))(*[_p(t) for t in outputs])
        check(lib().chelis_dag_run(self.handle, ins, len(inputs), outs, len(outputs)), "dag run")
        if self.has_traps:
            # the earliest failing launch's lowest failing element, read once
            # after the run (a synchronization)
            failure = take_numeric_failure()
            if failure:
                raise ChelisError(failure[2])
        if self.has_count:
            # the trap channel, read once after the run (a synchronization)
            if trap_status():
                raise ChelisError("numeric trap: domain in count at bool")
        return outputs


def dag_fuse(json_text: str) -> str:
    """fuse.rs alone: the DAG after greedy chain fusion, in the wire form."""
    data = json_text.encode()
    out = lib().chelis_dag_fuse(data, len(data))
    if out is None:
        raise ChelisError(lib().chelis_hip_last_error().decode(errors="replace"))
    return out.decode()


def prepare_dag_for_codegen(json_text: str) -> str:
    """The BLAS selection before codegen (lowered matmuls as BlasMatmul)."""
    data = json_text.encode()
    out = lib().chelis_prepare_dag_for_codegen(data, len(data))
    if out is None:
        raise ChelisError(lib().chelis_hip_last_error().decode(errors="replace"))
    return out.decode()


def tensor_capable_prims():
    """TENSOR_CAPABLE_PRIMS as dtype ids."""
    arr = POINTER(c_uint8)()
    n = lib().chelis_hip_tensor_capable_prims(ctypes.byref(arr))
    return [arr[k] for k in range(n)]


def runtime_dir() -> str:
    return lib().chelis_hip_runtime_dir().decode()


def codegen_hip_host_program(helpers):
    """[(name, dag_json)] -> [(name, CodegenResult)] for the Count-bearing helpers."""
    names = (ctypes.c_char_p * max(1, len(helpers)))(*[n.encode() for n, _ in helpers])
    texts = [t.encode() for _, t in helpers]
    dags = (ctypes.c_char_p * max(1, len(helpers)))(*texts)
    lens = (c_int64 * max(1, len(helpers)))(*[len(t) for t in texts])
    L = lib()
    h = L.chelis_codegen_hip_host_program(len(helpers), names, dags, lens)
    if not h:
        raise ChelisError("codegen_hip_host_program failed: " + L.chelis_hip_last_error().decode(errors="replace"))
    try:
        return [(L.chelis_host_program_helper_name(h, k).decode(),
                 CodegenResult._from_handle(L.chelis_host_program_helper(h, k)))
                for k in range(L.chelis_host_program_helper_count(h))]
    finally:
        L.chelis_host_program_release(h)


class CodegenResult:
    """chelis_codegen_hip: the HipCodegenResult fields."""

    @classmethod
    def _from_handle(cls, h):
        self = cls.__new__(cls)
        self._read(h)
        return self

    def __init__(self, json_text: str, func_name: str):
        data = json_text.encode()
        h = lib().chelis_codegen_hip(data, len(data), func_name.encode())
        if not h:
            raise ChelisError("codegen_hip failed: " + lib().chelis_hip_last_error().decode(errors="replace"))
        try:
            self._read(h)
        finally:
            lib().chelis_codegen_release(h)

    def _read(self, h):
        L = lib()
        lists = [[L.chelis_codegen_list_item(h, w, i).decode() for i in range(L.chelis_codegen_list_count(h, w))]
                 for w in range(5)]
        self.c_source = L.chelis_codegen_c_source(h).decode()
        self.h_header = L.chelis_codegen_h_header(h).decode()
        self.compile_flags, self.link_flags, self.input_labels, self.output_labels, self.symbolic_dims = lists
        self.peak_device_bytes_formula = L.chelis_codegen_peak_device_bytes_formula(h).decode()
        est = L.chelis_codegen_peak_device_bytes_estimate(h)
        self.peak_device_bytes_estimate = None if est < 0 else est


class GeneratedProgram:
    """chelis_codegen_hip's source compiled with its own compile and link
    flags into `directory` and loaded: the generated {f}_device and {f}
    entries, as the reference's Python binding loads a built module
    (crates/chelis-python/src/lib.rs:406-441)."""

    def __init__(self, json_text: str, func_name: str, directory: str, compiler: str = "g++"):
        self.result = CodegenResult(json_text, func_name)
        self.name = func_name
        src = os.path.join(directory, func_name + ".cpp")
        with open(src, "w") as fh:
            fh.write(self.result.c_source)
        self.path = os.path.join(directory, "lib" + func_name + ".so")
        cmd = [compiler, "-shared", "-fPIC", *self.result.compile_flags, src, "-o", self.path,
               *self.result.link_flags]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise ChelisError("generated source failed to build:\n" + r.stderr[-4000:])
        lib()  # the library the generated code links is loaded first, from this tree
        self.library = ctypes.CDLL(self.path)
        self.n_out = len(self.result.output_labels)

    def device(self, inputs):
        """{f}_device over owned device tensors; returns the owned outputs."""
        return device_entry(self.name, inputs, self.n_out, self.library)

    def host(self, arrays):
        """{f} over numpy arrays (host tensors in and out)."""
        return host_entry(self.name, arrays, self.n_out, self.library)

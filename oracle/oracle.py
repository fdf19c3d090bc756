"""ctypes view of the CPU oracle (liboracle.so): TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker or the timed CPU baseline. The product
package (chelis_amd) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build() -> None:
    """Compile the oracle (and, where /root/reference exists, oracle/_ref)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


c_i64, c_u64, c_f32, c_f64, c_p = ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_double, ctypes.c_void_p


def _declare(L):
    sig = {
        "orc_set_threads": (ctypes.c_int, [ctypes.c_int]),
        "orc_splitmix64": (c_u64, [c_u64]),
        "orc_derive": (c_u64, [c_u64, c_u64]),
        "orc_word": (c_u64, [c_u64, c_u64]),
        "orc_unit": (c_f64, [c_u64, c_u64]),
        "orc_split": (None, [c_u64, c_p]),
        "orc_fold_in": (c_u64, [c_u64, c_i64]),
        "orc_split_n": (None, [c_u64, c_i64, c_p]),
        "orc_uniform_like_f32": (None, [c_u64, c_f32, c_f32, c_p, c_i64]),
        "orc_uniform_like_f64": (None, [c_u64, c_f64, c_f64, c_p, c_i64]),
        "orc_expf": (c_f32, [c_f32]), "orc_exp": (c_f64, [c_f64]),
        "orc_logf": (c_f32, [c_f32]), "orc_log": (c_f64, [c_f64]),
        "orc_erfcf": (c_f32, [c_f32]), "orc_erfc": (c_f64, [c_f64]),
        "orc_tanhf": (c_f32, [c_f32]), "orc_tanh": (c_f64, [c_f64]),
        "orc_tree_sum_f32": (c_f32, [c_p, c_i64, c_i64]),
        "orc_tree_sum_f64": (c_f64, [c_p, c_i64, c_i64]),
        "orc_level_sum_f32": (c_f32, [c_p, c_i64]),
        "orc_level_sum_f64": (c_f64, [c_p, c_i64]),
        "orc_max_reduce_f32": (c_f32, [c_p, c_i64, c_i64]),
        "orc_max_reduce_f64": (c_f64, [c_p, c_i64, c_i64]),
        "orc_sum_axis_f32": (None, [c_p, c_i64, c_i64, c_i64, c_p]),
        "orc_sum_axis_f64": (None, [c_p, c_i64, c_i64, c_i64, c_p]),
        "orc_max_axis_f32": (None, [c_p, c_i64, c_i64, c_i64, c_p]),
        "orc_max_axis_f64": (None, [c_p, c_i64, c_i64, c_i64, c_p]),
        "orc_prod_axis_f32": (None, [c_p, c_i64, c_i64, c_i64, c_p]),
        "orc_prod_axis_f64": (None, [c_p, c_i64, c_i64, c_i64, c_p]),
        "orc_count_axis": (ctypes.c_int32, [c_p, c_i64, c_i64, c_i64, c_p]),
        "orc_softmax_rows_f32": (None, [c_p, c_p, c_i64, c_i64]),
        "orc_softmax_rows_f64": (None, [c_p, c_p, c_i64, c_i64]),
        "orc_softmax_adjoint_rows_f32": (None, [c_p, c_p, c_p, c_i64, c_i64]),
        "orc_softmax_adjoint_rows_f64": (None, [c_p, c_p, c_p, c_i64, c_i64]),
        "orc_layer_norm_rows_f32": (None, [c_p, c_p, c_p, c_f32, c_p, c_i64, c_i64]),
        "orc_layer_norm_rows_f64": (None, [c_p, c_p, c_p, c_f64, c_p, c_i64, c_i64]),
        "orc_gelu_f32": (None, [c_p, c_p, c_i64]),
        "orc_gelu_f64": (None, [c_p, c_p, c_i64]),
        "orc_relu_f32": (None, [c_p, c_p, c_i64]),
        "orc_relu_adjoint_f32": (None, [c_p, c_p, c_p, c_i64]),
        "orc_dropout_f32": (None, [c_u64, c_p, c_f32, c_p, c_i64]),
        "orc_dropout_replay_f32": (None, [c_u64, c_p, c_f32, c_p, c_i64]),
        "orc_dropout_f64": (None, [c_u64, c_p, c_f64, c_p, c_i64]),
        "orc_dropout_replay_f64": (None, [c_u64, c_p, c_f64, c_p, c_i64]),
        "orc_matmul_f32": (None, [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_i64]),
        "orc_matmul_f64": (None, [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_i64]),
        "orc_linreg_step_f64": (None, [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64]),
        "orc_narrow_decode": (None, [ctypes.c_int, c_p, c_p, c_i64]),
        "orc_narrow_encode": (None, [ctypes.c_int, c_p, c_p, c_i64]),
        "orc_narrow_sub": (None, [ctypes.c_int, c_p, c_p, c_p, c_i64]),
        "orc_narrow_max": (None, [ctypes.c_int, c_p, c_p, c_p, c_i64]),
        "orc_narrow_min": (None, [ctypes.c_int, c_p, c_p, c_p, c_i64]),
        "orc_narrow_relu": (None, [ctypes.c_int, c_p, c_p, c_i64]),
        "orc_narrow_relu_adjoint": (None, [ctypes.c_int, c_p, c_p, c_p, c_i64]),
        "orc_matmul_narrow": (None, [ctypes.c_int, c_p, c_p, c_p, c_i64, c_i64, c_i64]),
        "orc_transformer_block_f32": (None, [c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_i64]),
        "orc_mlp_train_step_f32": (None, [c_p, c_p, c_p, c_p, c_p, c_p, c_u64, c_f32, c_f32, c_p,
                                          c_i64, c_i64, c_i64, c_i64]),
    }
    sig.update({
        "orc_compare": (None, [ctypes.c_int, ctypes.c_int, c_p, c_p, c_p, c_i64]),
        "orc_logical": (None, [ctypes.c_int, c_p, c_p, c_p, c_i64]),
        "orc_where": (None, [c_p, c_p, c_p, c_p, c_i64, c_i64]),
        "orc_cast": (c_i64, [ctypes.c_int, ctypes.c_int, c_p, c_p, c_i64, c_p]),
        "orc_extrema_adjoint": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int, c_p, c_p, c_p, c_p, c_i64]),
        "orc_int_binary": (c_i64, [ctypes.c_int, ctypes.c_int, c_p, c_p, c_p, c_i64, c_p]),
        "orc_int_unary": (c_i64, [ctypes.c_int, ctypes.c_int, c_p, c_p, c_i64, c_p]),
        "orc_cumsum": (c_i64, [ctypes.c_int, c_p, c_p, c_i64, c_i64, c_i64, ctypes.c_int, c_p]),
        "orc_pad": (None, [ctypes.c_int, c_p, ctypes.c_int, c_p, c_p, c_p, ctypes.c_uint64, c_p]),
        "orc_slice": (None, [ctypes.c_int, c_p, ctypes.c_int, c_p, c_p, c_p, c_p, c_p]),
        "orc_scatter": (c_i64, [ctypes.c_int, ctypes.c_int, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_i64,
                                c_p]),
        "orc_scatter_elements": (c_i64, [ctypes.c_int, c_p, c_p, c_p, c_p, ctypes.c_int, c_p, c_p, ctypes.c_int,
                                         c_p]),
        "orc_gather": (c_i64, [c_p, c_i64, c_i64, c_i64, c_i64, c_p, ctypes.c_int, c_i64, c_i64, c_p, c_p]),
    })
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f(dtype):
    return "f32" if np.dtype(dtype) == np.float32 else "f64"


# ---- RNG ----
def split(key: int) -> tuple[int, int]:
    out = np.zeros(2, np.uint64)
    lib().orc_split(key & (2**64 - 1), _ptr(out))
    return int(out[0]), int(out[1])


def fold_in(key: int, n: int) -> int:
    return int(lib().orc_fold_in(key & (2**64 - 1), n))


def split_n(key: int, n: int) -> list[int]:
    out = np.zeros(max(n, 1), np.uint64)
    lib().orc_split_n(key & (2**64 - 1), n, _ptr(out))
    return [int(v) for v in out[:n]]


def unit(key: int, index: int) -> float:
    return float(lib().orc_unit(key & (2**64 - 1), index))


def uniform_like(key: int, low, high, n: int, dtype=np.float32) -> np.ndarray:
    out = np.empty(n, dtype)
    getattr(lib(), f"orc_uniform_like_{_f(dtype)}")(key & (2**64 - 1), low, high, _ptr(out), n)
    return out


# ---- reductions ----
def tree_sum(x: np.ndarray) -> np.floating:
    x = np.ascontiguousarray(x)
    return x.dtype.type(getattr(lib(), f"orc_tree_sum_{_f(x.dtype)}")(_ptr(x), x.size, 1))


def level_sum(x: np.ndarray) -> np.floating:
    x = np.ascontiguousarray(x)
    return x.dtype.type(getattr(lib(), f"orc_level_sum_{_f(x.dtype)}")(_ptr(x), x.size))


def _axis_view(x: np.ndarray, axis: int):
    axis = axis % x.ndim
    outer = int(np.prod(x.shape[:axis], dtype=np.int64))
    inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
    return outer, x.shape[axis], inner, x.shape[:axis] + x.shape[axis + 1:]


def sum_axis(x: np.ndarray, axis: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    outer, n, inner, shape = _axis_view(x, axis)
    out = np.empty(shape, x.dtype)
    getattr(lib(), f"orc_sum_axis_{_f(x.dtype)}")(_ptr(x), outer, n, inner, _ptr(out))
    return out


def max_axis(x: np.ndarray, axis: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    outer, n, inner, shape = _axis_view(x, axis)
    out = np.empty(shape, x.dtype)
    getattr(lib(), f"orc_max_axis_{_f(x.dtype)}")(_ptr(x), outer, n, inner, _ptr(out))
    return out


def prod_axis(x: np.ndarray, axis: int) -> np.ndarray:
    """ProdReduce: the C lane's left fold from 1 over `axis`."""
    x = np.ascontiguousarray(x)
    outer, n, inner, shape = _axis_view(x, axis)
    out = np.empty(shape, x.dtype)
    getattr(lib(), f"orc_prod_axis_{_f(x.dtype)}")(_ptr(x), outer, n, inner, _ptr(out))
    return out


def count_axis(x: np.ndarray, axis: int):
    x = np.ascontiguousarray(x, dtype=np.uint8)
    outer, n, inner, shape = _axis_view(x, axis)
    out = np.empty(shape, np.int64)
    err = lib().orc_count_axis(_ptr(x), outer, n, inner, _ptr(out))
    return out, int(err)


# ---- row regions / elementwise ----
def softmax_rows(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    n = x.shape[-1]
    getattr(lib(), f"orc_softmax_rows_{_f(x.dtype)}")(_ptr(x), _ptr(y), x.size // max(n, 1), n)
    return y


def softmax_adjoint_rows(y, g) -> np.ndarray:
    y = np.ascontiguousarray(y)
    g = np.ascontiguousarray(g, y.dtype)
    dx = np.empty_like(y)
    n = y.shape[-1]
    getattr(lib(), f"orc_softmax_adjoint_rows_{_f(y.dtype)}")(_ptr(y), _ptr(g), _ptr(dx), y.size // n, n)
    return dx


def layer_norm_rows(x, gamma, beta, eps) -> np.ndarray:
    x = np.ascontiguousarray(x)
    g = np.ascontiguousarray(gamma, x.dtype)
    b = np.ascontiguousarray(beta, x.dtype)
    y = np.empty_like(x)
    n = x.shape[-1]
    getattr(lib(), f"orc_layer_norm_rows_{_f(x.dtype)}")(_ptr(x), _ptr(g), _ptr(b), eps, _ptr(y),
                                                          x.size // n, n)
    return y


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    getattr(lib(), f"orc_gelu_{_f(x.dtype)}")(_ptr(x), _ptr(y), x.size)
    return y


def relu(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_relu_f32(_ptr(x), _ptr(y), x.size)
    return y


def relu_adjoint(x, g) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(g, np.float32)
    y = np.empty_like(x)
    lib().orc_relu_adjoint_f32(_ptr(x), _ptr(g), _ptr(y), x.size)
    return y


def dropout(key: int, x: np.ndarray, rate) -> np.ndarray:
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    getattr(lib(), f"orc_dropout_{_f(x.dtype)}")(key & (2**64 - 1), _ptr(x), rate, _ptr(y), x.size)
    return y


def dropout_replay(key: int, g: np.ndarray, rate) -> np.ndarray:
    """The forward mask on the cotangent, kept values divided by (1 - rate),
    at g's dtype (binary32 unless g is binary64)."""
    g = np.ascontiguousarray(g, np.float64 if np.asarray(g).dtype == np.float64 else np.float32)
    y = np.empty_like(g)
    getattr(lib(), f"orc_dropout_replay_{_f(g.dtype)}")(key & (2**64 - 1), _ptr(g), rate, _ptr(y), g.size)
    return y


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Canonical-tree matmul of 2-D arrays (any strides, via element strides)."""
    assert a.dtype == b.dtype and a.ndim == 2 and b.ndim == 2 and a.shape[1] == b.shape[0]
    isz = a.dtype.itemsize
    M, K = a.shape
    N = b.shape[1]
    c = np.empty((M, N), a.dtype)
    getattr(lib(), f"orc_matmul_{_f(a.dtype)}")(
        a.ctypes.data, a.strides[0] // isz, a.strides[1] // isz,
        b.ctypes.data, b.strides[0] // isz, b.strides[1] // isz, _ptr(c), M, N, K)
    return c


def unary(name: str, x: np.ndarray) -> np.ndarray:
    fn = getattr(lib(), f"orc_{name}{'f' if x.dtype == np.float32 else ''}")
    return np.array([fn(v) for v in x.ravel()], x.dtype).reshape(x.shape)


# ---- programs ----
# ---- bfloat16 / binary16 storage (16-bit carriers as np.uint16 bit patterns) ----
NARROW = {"bf16": 0, "f16": 1}


def narrow_decode(kind: str, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    y = np.empty(x.shape, np.float32)
    lib().orc_narrow_decode(NARROW[kind], _ptr(x), _ptr(y), x.size)
    return y


def narrow_encode(kind: str, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_narrow_encode(NARROW[kind], _ptr(x), _ptr(y), x.size)
    return y


def narrow_binary(op: str, kind: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    y = np.empty(a.shape, np.uint16)
    getattr(lib(), f"orc_narrow_{op}")(NARROW[kind], _ptr(a), _ptr(b), _ptr(y), a.size)
    return y


def narrow_relu(kind: str, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    y = np.empty(x.shape, np.uint16)
    lib().orc_narrow_relu(NARROW[kind], _ptr(x), _ptr(y), x.size)
    return y


def narrow_relu_adjoint(kind: str, x: np.ndarray, g: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    g = np.ascontiguousarray(g, np.uint16)
    y = np.empty(x.shape, np.uint16)
    lib().orc_narrow_relu_adjoint(NARROW[kind], _ptr(x), _ptr(g), _ptr(y), x.size)
    return y


def narrow_matmul(kind: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    M, K = a.shape
    N = b.shape[1]
    c = np.empty((M, N), np.uint16)
    lib().orc_matmul_narrow(NARROW[kind], _ptr(a), _ptr(b), _ptr(c), M, N, K)
    return c


def linreg_step(X, w, y):
    X = np.ascontiguousarray(X, np.float64)
    w = np.ascontiguousarray(w, np.float64)
    y = np.ascontiguousarray(y, np.float64)
    n, d = X.shape
    grad = np.empty(d, np.float64)
    loss = np.empty(1, np.float64)
    lib().orc_linreg_step_f64(_ptr(X), _ptr(w), _ptr(y), _ptr(grad), _ptr(loss), n, d)
    return grad, loss[0]


TRANSFORMER_PARAMS = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
                      "ln2_g", "ln2_b", "w1", "b1", "w2", "b2")


def transformer_block(x, params: dict, heads: int):
    x = np.ascontiguousarray(x, np.float32)
    batch, seq, dm = x.shape
    ffn = params["w1"].shape[1]
    arrs = [np.ascontiguousarray(params[k], np.float32) for k in TRANSFORMER_PARAMS]
    ptrs = (ctypes.c_void_p * 16)(*[a.ctypes.data for a in arrs])
    out = np.empty_like(x)
    lib().orc_transformer_block_f32(_ptr(x), ctypes.cast(ptrs, ctypes.c_void_p), _ptr(out),
                                    batch, seq, dm, heads, ffn)
    return out


def mlp_train_step(x, onehot, w1, b1, w2, b2, key, rate, lr):
    """Returns (loss, w1', b1', w2', b2'); inputs are not modified."""
    x = np.ascontiguousarray(x, np.float32)
    onehot = np.ascontiguousarray(onehot, np.float32)
    w1, b1, w2, b2 = (np.array(a, np.float32, copy=True) for a in (w1, b1, w2, b2))
    loss = np.empty(1, np.float32)
    B, din = x.shape
    dh, dout = w2.shape
    lib().orc_mlp_train_step_f32(_ptr(x), _ptr(onehot), _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2),
                                 key & (2**64 - 1), rate, lr, _ptr(loss), B, din, dh, dout)
    return loss[0], w1, b1, w2, b2


# ---- comparison, logical, where, checked cast / integer arithmetic, gather ----
# Dtype names and the device packet's ids; bf16 / f16 travel as np.uint16
# bit patterns, bool as one byte per element.
DTYPE_IDS = {"f32": 0, "f64": 1, "i32": 2, "bool": 3, "i64": 4, "bf16": 5, "f16": 6, "i8": 7, "i16": 8}
CARRIERS = {"f32": np.float32, "f64": np.float64, "i32": np.int32, "bool": np.uint8, "i64": np.int64,
            "bf16": np.uint16, "f16": np.uint16, "i8": np.int8, "i16": np.int16}
COMPARE_KINDS = {"cmp_lt": 0, "lt": 1, "eq": 2, "neq": 3, "gt": 4, "gte": 5, "lte": 6}
LOGICAL_KINDS = {"and": 0, "or": 1, "not": 2}
INT_BINARY = {"add": 0, "sub": 1, "mul": 2, "floor_div": 3, "trunc_div": 4, "mod": 5, "max_elem": 6, "min_elem": 7,
              "bitand": 8, "bitor": 9, "bitxor": 10, "shl": 11, "shr": 12}
INT_UNARY = {"neg": 0, "abs": 1}
FAILURE_KINDS = {1: "overflow", 2: "domain", 3: "division by zero"}


def _carrier(dt: str, a) -> np.ndarray:
    a = np.asarray(a)
    if dt == "f16" and a.dtype == np.float16:
        a = a.view(np.uint16)
    return np.ascontiguousarray(a, CARRIERS[dt])


def _broadcast(*arrays):
    shape = np.broadcast_shapes(*[a.shape for a in arrays])
    return shape, [np.ascontiguousarray(np.broadcast_to(a, shape)) for a in arrays]


def trap_text(kind: int, op: str, dt: str) -> str:
    """[04-NUM-9]'s rendering of a failure (spec/04-type-system.md:3896-3898)."""
    return f"numeric trap: {FAILURE_KINDS[kind]} in {op} at {dt}"


def compare(kind: str, dt: str, a, b) -> np.ndarray:
    """Bool8 result of one comparison; operands broadcast (numpy rules)."""
    shape, (a, b) = _broadcast(_carrier(dt, a), _carrier(dt, b))
    out = np.empty(shape, np.uint8)
    lib().orc_compare(COMPARE_KINDS[kind], DTYPE_IDS[dt], _ptr(a), _ptr(b), _ptr(out), out.size)
    return out


def logical(kind: str, a, b=None) -> np.ndarray:
    a = _carrier("bool", a)
    if b is None:
        b = a
    shape, (a, b) = _broadcast(a, _carrier("bool", b))
    out = np.empty(shape, np.uint8)
    lib().orc_logical(LOGICAL_KINDS[kind], _ptr(a), _ptr(b), _ptr(out), out.size)
    return out


def where(cond, a, b) -> np.ndarray:
    """The selected operand's stored bytes; a and b share one numpy dtype."""
    a, b = np.asarray(a), np.asarray(b)
    shape, (c, a, b) = _broadcast(_carrier("bool", cond), a, b.astype(a.dtype, copy=False))
    out = np.empty(shape, a.dtype)
    lib().orc_where(_ptr(c), _ptr(a), _ptr(b), _ptr(out), a.dtype.itemsize, out.size)
    return out


def extrema_adjoint(kind: str, operand: str, dt: str, a, b, g) -> np.ndarray:
    """kind "max" / "min", operand "left" / "right"; operands broadcast."""
    shape, (a, b, g) = _broadcast(_carrier(dt, a), _carrier(dt, b), _carrier(dt, g))
    out = np.empty(shape, CARRIERS[dt])
    lib().orc_extrema_adjoint(int(kind == "min"), int(operand == "right"), DTYPE_IDS[dt], _ptr(a), _ptr(b), _ptr(g),
                              _ptr(out), out.size)
    return out


def cast(src: str, dst: str, x):
    """(result, first failing index or -1, failure kind)."""
    x = _carrier(src, x)
    y = np.empty(x.shape, CARRIERS[dst])
    kind = ctypes.c_int32(0)
    first = lib().orc_cast(DTYPE_IDS[src], DTYPE_IDS[dst], _ptr(x), _ptr(y), x.size, ctypes.byref(kind))
    return y, first, kind.value


def int_binary(op: str, dt: str, a, b):
    """(result, first failing index or -1, failure kind); operands broadcast."""
    shape, (a, b) = _broadcast(_carrier(dt, a), _carrier(dt, b))
    y = np.empty(shape, CARRIERS[dt])
    kind = ctypes.c_int32(0)
    first = lib().orc_int_binary(INT_BINARY[op], DTYPE_IDS[dt], _ptr(a), _ptr(b), _ptr(y), y.size,
                                 ctypes.byref(kind))
    return y, first, kind.value


def int_unary(op: str, dt: str, x):
    x = _carrier(dt, x)
    y = np.empty(x.shape, CARRIERS[dt])
    kind = ctypes.c_int32(0)
    first = lib().orc_int_unary(INT_UNARY[op], DTYPE_IDS[dt], _ptr(x), _ptr(y), x.size, ctypes.byref(kind))
    return y, first, kind.value


def gather_shape(vshape, ishape, axis: int, batch_rank: int):
    return tuple(vshape[:axis]) + tuple(ishape[batch_rank:]) + tuple(vshape[axis + 1:])


def gather(values: np.ndarray, indices: np.ndarray, axis: int, batch_rank: int = 0):
    """(result, first failing index or -1, failure kind): RiscOp::Gather with
    the reference HIP lane's geometry. The leading batch_rank axes of values
    and indices must match (the host-side domain check)."""
    values = np.ascontiguousarray(values)
    indices = np.ascontiguousarray(indices)
    assert indices.dtype in (np.int32, np.int64)
    assert tuple(values.shape[:batch_rank]) == tuple(indices.shape[:batch_rank])
    axis_size = values.shape[axis]
    after = int(np.prod(values.shape[axis + 1:], dtype=np.int64))
    before = int(np.prod(values.shape[:axis], dtype=np.int64))
    batch = int(np.prod(values.shape[:batch_rank], dtype=np.int64))
    index_count = 0 if batch == 0 else indices.size // batch
    out = np.empty(gather_shape(values.shape, indices.shape, axis, batch_rank), values.dtype)
    kind = ctypes.c_int32(0)
    first = lib().orc_gather(_ptr(values), values.dtype.itemsize, before, axis_size, after, _ptr(indices),
                             2 if indices.dtype == np.int32 else 4, index_count, batch, _ptr(out),
                             ctypes.byref(kind))
    return out, first, kind.value


def cumsum(dt: str, x, axis: int, reverse: bool = False):
    """(result, first failing position in the evaluation order or -1, kind):
    [05-OP-33]'s ordered scan, the C lane's accumulation. i8 / i16 scan into
    i32."""
    x = _carrier(dt, x)
    ax = axis % x.ndim
    outer = int(np.prod(x.shape[:ax], dtype=np.int64))
    inner = int(np.prod(x.shape[ax + 1:], dtype=np.int64))
    rdt = "i32" if dt in ("i8", "i16") else dt
    y = np.empty(x.shape, CARRIERS[rdt])
    kind = ctypes.c_int32(0)
    first = lib().orc_cumsum(DTYPE_IDS[dt], _ptr(x), _ptr(y), outer, x.shape[ax], inner, int(reverse),
                             ctypes.byref(kind))
    return y, first, kind.value


def _i64s(v):
    return np.ascontiguousarray(np.asarray(v, np.int64).reshape(-1))


def pad(x, lo, hi, fill):
    """RiscOp::Pad over any dtype: `fill` a scalar of x's dtype (a 16-bit
    float as its bits in x's carrier)."""
    x = np.ascontiguousarray(x)
    lo, hi = _i64s(lo), _i64s(hi)
    out_shape = _i64s([e + a + b for e, a, b in zip(x.shape, lo, hi)])
    y = np.empty(tuple(out_shape), x.dtype)
    bits = int(np.array([fill], x.dtype).view(np.dtype("u%d" % x.itemsize))[0])
    src = _i64s(x.shape)
    lib().orc_pad(x.itemsize, _ptr(x), x.ndim, _ptr(src), _ptr(lo), _ptr(out_shape), bits, _ptr(y))
    return y


def slice_(x, start, step, out_shape):
    """RiscOp::Shrink (step 1) / RiscOp::Stride (start 0): element o reads
    x at o * step + start."""
    x = np.ascontiguousarray(x)
    start, step, out_shape = _i64s(start), _i64s(step), _i64s(out_shape)
    y = np.empty(tuple(out_shape), x.dtype)
    src = _i64s(x.shape)
    lib().orc_slice(x.itemsize, _ptr(x), x.ndim, _ptr(src), _ptr(start), _ptr(step), _ptr(out_shape), _ptr(y))
    return y


def scatter(dt: str, target, indices, updates, axis: int, batch_rank: int = 0, add: bool = False):
    """RiscOp::ScatterAdd (add) / Scatter: (result, first failing position
    or -1, kind); updates have the gathered shape target[..axis] ++
    indices[batch_rank..] ++ target[axis+1..]. A domain failure's position
    is the update's; an overflow's is the update count + the destination."""
    target = _carrier(dt, target)
    updates = _carrier(dt, updates)
    idx = np.ascontiguousarray(indices, np.int64)
    assert updates.shape == gather_shape(target.shape, idx.shape, axis, batch_rank), "updates shape"
    batch = int(np.prod(target.shape[:batch_rank], dtype=np.int64))
    before = int(np.prod(target.shape[:axis], dtype=np.int64))
    after = int(np.prod(target.shape[axis + 1:], dtype=np.int64))
    index_count = idx.size // batch if batch else 0
    opb = before // batch if batch and before else 1
    out = np.empty_like(target)
    kind = ctypes.c_int32(0)
    first = lib().orc_scatter(int(add), DTYPE_IDS[dt], _ptr(target), _ptr(idx), _ptr(updates), _ptr(out), before,
                              target.shape[axis], after, index_count, opb, ctypes.byref(kind))
    return out, first, kind.value


def scatter_elements(dt: str, data, indices, updates, axis: int):
    """RiscOp::ScatterElements: (result, first failing position or -1, kind)."""
    data = _carrier(dt, data)
    updates = _carrier(dt, updates)
    idx = np.ascontiguousarray(indices, np.int64)
    assert updates.shape == idx.shape and idx.ndim == data.ndim
    out = np.empty_like(data)
    kind = ctypes.c_int32(0)
    ishape, dshape = _i64s(idx.shape), _i64s(data.shape)  # held for the call
    first = lib().orc_scatter_elements(DTYPE_IDS[dt], _ptr(data), _ptr(idx), _ptr(updates), _ptr(out), data.ndim,
                                       _ptr(ishape), _ptr(dshape), axis, ctypes.byref(kind))
    return out, first, kind.value

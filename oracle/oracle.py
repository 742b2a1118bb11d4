"""ORACLE (test infrastructure only): ctypes access to the CPU restatement
(liboracle.so, built from spinn_cpu.c + cpu_runtime.c) and, where it was
built, to the reference's own CPU runtime (_ref/libspinn_ref.so).

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use
this module, and only as the parity reference / the timed CPU baseline.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libspinn_ref.so"
REF_SRC = Path("/root/reference/SPINN")

_FP = C.POINTER(C.c_float)
_DP = C.POINTER(C.c_double)


class OracleConv(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "n", "c", "h", "w", "oc", "oh", "ow", "kh", "kw", "sh", "sw", "ph", "pw", "group", "act")]


def build(ref: bool = True) -> None:
    """Compile liboracle.so and, when the reference sources are present, _ref/libspinn_ref.so and
    _ref/onnx2ennf."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if ref and REF_SRC.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "-j8", "ref"], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build(ref=False)
        L = C.CDLL(str(LIB))
        L.oracle_conv2d.argtypes = [C.POINTER(OracleConv), _FP, _FP, _FP, _FP, _FP]
        L.oracle_conv2d_f64.argtypes = [C.POINTER(OracleConv), _FP, _FP, _FP, _FP, _DP]
        L.oracle_winograd.argtypes = [C.POINTER(OracleConv), _FP, _FP, _FP, _FP, _FP]
        L.oracle_gemm.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, _FP, _FP, _FP,
                                  C.c_int, _FP]
        L.oracle_gemm_f64.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double, C.c_double, _FP, _FP,
                                      _FP, C.c_int, _DP]
        L.oracle_matmul.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, _FP, _FP, _FP]
        L.oracle_maxpool.argtypes = [C.c_int] * 12 + [_FP, _FP]
        L.oracle_reduce_mean.argtypes = [C.c_long, C.c_long, C.c_long, _FP, _FP]
        L.oracle_set_as_shipped.argtypes = [C.c_int]
        L.oracle_set_num_threads.argtypes = [C.c_int]
        L.oracle_model_load.restype = C.c_void_p
        L.oracle_model_load.argtypes = [C.c_char_p]
        L.oracle_model_run.argtypes = [C.c_void_p, _FP, _FP]
        L.oracle_model_free.argtypes = [C.c_void_p]
        L.oracle_model_tensor.restype = C.c_long
        L.oracle_model_tensor.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]
        L.oracle_model_set_winograd.argtypes = [C.c_void_p, C.c_int]
        L.oracle_model_num_nodes.argtypes = [C.c_void_p]
        L.oracle_binary.argtypes = [C.c_int, _FP, C.c_uint32, _FP, C.c_uint32, _FP, C.c_uint32]
        L.oracle_unary.argtypes = [C.c_int, _FP, _FP, C.c_long]
        L.oracle_batchnorm.argtypes = [C.c_long, C.c_long, C.c_long, _FP, _FP, _FP, _FP, _FP, C.c_float, _FP]
        L.oracle_softmax.argtypes = [C.c_long, C.c_long, C.c_long, _FP, _FP]
        L.oracle_concat.argtypes = [C.c_int, C.POINTER(_FP), C.POINTER(C.c_long), C.c_long, C.c_long, _FP]
        L.oracle_split.argtypes = [C.c_int, C.POINTER(_FP), C.POINTER(C.c_long), C.c_long, C.c_long, _FP]
        L.oracle_transpose.argtypes = [C.c_int, C.POINTER(C.c_long), C.POINTER(C.c_int), _FP, _FP]
        L.oracle_resize_nearest.argtypes = [C.c_long, C.c_int, C.c_int, C.c_int, C.c_int, _FP, _FP]
        _lib = L
    return _lib


def _f(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_FP)


def conv_desc(n, c, h, w, oc, kh, kw, sh=1, sw=1, ph=0, pw=0, group=1, act=0, oh=None, ow=None) -> OracleConv:
    if oh is None:
        oh = (h + 2 * ph - kh) // sh + 1
    if ow is None:
        ow = (w + 2 * pw - kw) // sw + 1
    return OracleConv(n, c, h, w, oc, oh, ow, kh, kw, sh, sw, ph, pw, group, act)


def conv2d(d: OracleConv, x, w, bias=None, res=None, as_shipped=False) -> np.ndarray:
    """Restated SPINN conv (float32, im2col + packed 6x16 GEMM + epilogue)."""
    y = np.zeros((d.n, d.oc, d.oh, d.ow), np.float32)
    L = lib()
    L.oracle_set_as_shipped(1 if as_shipped else 0)
    try:
        rc = L.oracle_conv2d(C.byref(d), _f(x), _f(w), _f(bias), _f(res), _f(y))
    finally:
        L.oracle_set_as_shipped(0)
    assert rc == 0
    return y


def conv2d_f64(d: OracleConv, x, w, bias=None, res=None) -> np.ndarray:
    """Closed-form direct convolution accumulated in float64, with the epilogue."""
    y = np.zeros((d.n, d.oc, d.oh, d.ow), np.float64)
    rc = lib().oracle_conv2d_f64(C.byref(d), _f(x), _f(w), _f(bias), _f(res), y.ctypes.data_as(_DP))
    assert rc == 0
    return y


def winograd(d: OracleConv, x, w, bias=None, res=None) -> np.ndarray:
    y = np.zeros((d.n, d.oc, d.oh, d.ow), np.float32)
    rc = lib().oracle_winograd(C.byref(d), _f(x), _f(w), _f(bias), _f(res), _f(y))
    assert rc == 0
    return y


def gemm(a, b, c=None, alpha=1.0, beta=1.0, trans_a=0, trans_b=0) -> np.ndarray:
    m = a.shape[1] if trans_a else a.shape[0]
    k = a.shape[0] if trans_a else a.shape[1]
    n = b.shape[0] if trans_b else b.shape[1]
    y = np.zeros((m, n), np.float32)
    rc = lib().oracle_gemm(m, n, k, trans_a, trans_b, alpha, beta, _f(a), _f(b), _f(c), 0 if c is None else c.size,
                           _f(y))
    assert rc == 0
    return y


def gemm_f64(a, b, c=None, alpha=1.0, beta=1.0, trans_a=0, trans_b=0) -> np.ndarray:
    m = a.shape[1] if trans_a else a.shape[0]
    k = a.shape[0] if trans_a else a.shape[1]
    n = b.shape[0] if trans_b else b.shape[1]
    y = np.zeros((m, n), np.float64)
    rc = lib().oracle_gemm_f64(m, n, k, trans_a, trans_b, alpha, beta, _f(a), _f(b), _f(c),
                               0 if c is None else c.size, y.ctypes.data_as(_DP))
    assert rc == 0
    return y


def matmul(a, b) -> np.ndarray:
    batch = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    m, k = a.shape[-2:]
    n = b.shape[-1]
    y = np.zeros(a.shape[:-2] + (m, n), np.float32)
    rc = lib().oracle_matmul(batch, m, n, k, _f(a), _f(b), _f(y))
    assert rc == 0
    return y


def maxpool(x, oh, ow, kh, kw, sh, sw, ph, pw) -> np.ndarray:
    n, c, h, w = x.shape
    y = np.zeros((n, c, oh, ow), np.float32)
    lib().oracle_maxpool(n, c, h, w, oh, ow, kh, kw, sh, sw, ph, pw, _f(x), _f(y))
    return y


def reduce_mean(x, outer, dim, inner) -> np.ndarray:
    y = np.zeros(outer * inner, np.float32)
    lib().oracle_reduce_mean(outer, dim, inner, _f(np.ascontiguousarray(x, np.float32)), _f(y))
    return y


BINARY_OPS = {"add": 0, "sub": 1, "mul": 2, "div": 3}
UNARY_OPS = {"relu": 0, "sigmoid": 1, "silu": 2}


def _c(a):
    return np.ascontiguousarray(a, np.float32)


def binary(op: str, a, b, out_shape) -> np.ndarray:
    """y[i] = a[i % a.size] op b[i % b.size] over prod(out_shape) outputs."""
    a, b = _c(a), _c(b)
    y = np.zeros(out_shape, np.float32)
    lib().oracle_binary(BINARY_OPS[op], _f(a), a.size, _f(b), b.size, _f(y), y.size)
    return y


def unary(op: str, x) -> np.ndarray:
    x = _c(x)
    y = np.zeros_like(x)
    lib().oracle_unary(UNARY_OPS[op], _f(x), _f(y), x.size)
    return y


def batchnorm(x, scale, bias, mean, var, eps=1e-5) -> np.ndarray:
    x = _c(x)
    y = np.zeros_like(x)
    spatial = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    lib().oracle_batchnorm(x.shape[0], x.shape[1], spatial, _f(x), _f(_c(scale)), _f(_c(bias)), _f(_c(mean)),
                           _f(_c(var)), eps, _f(y))
    return y


def _view(shape, axis):
    axis = axis % len(shape)
    return int(np.prod(shape[:axis])), int(np.prod(shape[axis + 1:])), axis


def softmax(x, axis=-1) -> np.ndarray:
    x = _c(x)
    y = np.zeros_like(x)
    outer, inner, axis = _view(x.shape, axis)
    lib().oracle_softmax(outer, x.shape[axis], inner, _f(x), _f(y))
    return y


def concat(xs, axis) -> np.ndarray:
    xs = [_c(x) for x in xs]
    outer, inner, axis = _view(xs[0].shape, axis)
    shape = list(xs[0].shape)
    shape[axis] = sum(x.shape[axis] for x in xs)
    y = np.zeros(shape, np.float32)
    ptrs = (_FP * len(xs))(*[_f(x) for x in xs])
    sizes = (C.c_long * len(xs))(*[x.shape[axis] for x in xs])
    lib().oracle_concat(len(xs), ptrs, sizes, outer, inner, _f(y))
    return y


def split(x, sizes, axis) -> list:
    x = _c(x)
    outer, inner, axis = _view(x.shape, axis)
    ys = []
    for s in sizes:
        shape = list(x.shape)
        shape[axis] = s
        ys.append(np.zeros(shape, np.float32))
    ptrs = (_FP * len(ys))(*[_f(y) for y in ys])
    lib().oracle_split(len(ys), ptrs, (C.c_long * len(sizes))(*sizes), outer, inner, _f(x))
    return ys


def transpose(x, perm) -> np.ndarray:
    x = _c(x)
    y = np.zeros([x.shape[p] for p in perm], np.float32)
    lib().oracle_transpose(x.ndim, (C.c_long * x.ndim)(*x.shape), (C.c_int * x.ndim)(*perm), _f(x), _f(y))
    return y


def resize_nearest(x, oh, ow) -> np.ndarray:
    x = _c(x)
    n, c, h, w = x.shape
    y = np.zeros((n, c, oh, ow), np.float32)
    lib().oracle_resize_nearest(n * c, h, w, oh, ow, _f(x), _f(y))
    return y


# ---- detector post-processing ----
_VP = C.c_void_p
_DT = {np.dtype(np.float32): 1, np.dtype(np.int32): 6, np.dtype(np.int64): 7}


def _vp(a):
    return C.c_void_p(a.ctypes.data)


def reduce_max(x, out_n) -> np.ndarray:
    """Max of each of out_n consecutive blocks of x (reduce_max.c)."""
    x = _c(x)
    y = np.zeros(out_n, np.float32)
    lib().oracle_reduce_max(C.c_uint32(out_n), C.c_uint32(x.size // out_n), _f(x), _f(y))
    return y


def topk(x, k):
    """Top-k along the last axis, sorted descending: (values fp32, indices int64)."""
    x = _c(x)
    n = x.shape[-1]
    rows = x.size // n if n else 0
    k = min(k, n)
    v = np.zeros(x.shape[:-1] + (k,), np.float32)
    i = np.zeros(x.shape[:-1] + (k,), np.int64)
    rc = lib().oracle_topk(C.c_long(rows), C.c_long(n), C.c_long(k), _f(x), _f(v), _vp(i))
    if rc:
        raise RuntimeError(rc)
    return v, i


def gather_elements(data, idx, axis) -> np.ndarray:
    data = _c(data)
    idx = np.ascontiguousarray(idx)
    axis %= data.ndim
    y = np.zeros(idx.shape, np.float32)
    u32 = C.c_uint32 * data.ndim
    lib().oracle_gather_elements(data.ndim, u32(*data.shape), u32(*idx.shape), axis, _f(data), _vp(idx),
                                 _DT[idx.dtype], _f(y), C.c_uint32(y.size))
    return y


def tile(x, out_shape) -> np.ndarray:
    x = np.ascontiguousarray(x)
    y = np.zeros(out_shape, x.dtype)
    u32 = C.c_uint32 * x.ndim
    lib().oracle_tile(x.ndim, u32(*x.shape), u32(*out_shape), x.dtype.itemsize, _vp(x), _vp(y))
    return y


def cast(x, dtype) -> np.ndarray:
    x = np.ascontiguousarray(x)
    y = np.zeros(x.shape, dtype)
    rc = lib().oracle_cast(_DT[x.dtype], _DT[y.dtype], C.c_uint32(x.size), _vp(x), _vp(y))
    if rc:
        raise RuntimeError(rc)
    return y


def binary_typed(op: str, a, b, out_shape) -> np.ndarray:
    """Integer Div / Mod (and float Mod) with the modulo broadcast."""
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    y = np.zeros(out_shape, a.dtype)
    rc = lib().oracle_binary_typed({"div": 3, "mod": 4}[op], _DT[a.dtype], _vp(a), C.c_uint32(a.size), _vp(b),
                                   C.c_uint32(b.size), _vp(y), C.c_uint32(y.size))
    if rc:
        raise RuntimeError(rc)
    return y


def set_threads(n: int) -> None:
    lib().oracle_set_num_threads(int(n))


class Model:
    """An ENNF model run on the CPU by the restated operators."""

    def __init__(self, path, winograd: bool = False):
        self._m = lib().oracle_model_load(str(path).encode())
        if not self._m:
            raise RuntimeError(f"oracle could not load {path}")
        lib().oracle_model_set_winograd(self._m, 1 if winograd else 0)

    def run(self, x: np.ndarray, out_shape, dtype=np.float32) -> np.ndarray:
        y = np.zeros(out_shape, dtype)
        rc = lib().oracle_model_run(self._m, _f(np.ascontiguousarray(x, np.float32)), C.cast(y.ctypes.data, _FP))
        if rc != 0:
            raise RuntimeError(f"oracle model run failed: {rc}")
        return y

    def tensor(self, tid: int, shape, dtype=np.float32) -> np.ndarray:
        a = np.zeros(shape, dtype)
        got = lib().oracle_model_tensor(self._m, tid, a.ctypes.data, a.nbytes)
        if got < 0:
            raise KeyError(tid)
        return a

    def close(self):
        if self._m:
            lib().oracle_model_free(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

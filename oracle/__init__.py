"""ctypes binding of the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY.  This restates the reference's CPU path
(``GQ.matvec`` / ``GQ.matmul`` / the block decoders; see okf_oracle.h for the
file:line each function follows and for what pins it).  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may use
it, and only as the checker or the timed CPU baseline -- never as the product.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_LIB = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        vp, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32
        lib.okf_ref_row_bytes.argtypes = [i32, u64, ctypes.POINTER(u64)]
        lib.okf_ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.okf_ref_f16_to_f32.restype = ctypes.c_float
        lib.okf_ref_dequant.argtypes = [i32, vp, u64, vp]
        lib.okf_ref_matvec.argtypes = [i32, vp, u32, u32, vp, vp, ctypes.c_int]
        lib.okf_ref_matmul.argtypes = [i32, vp, u32, u32, vp, u32, vp, ctypes.c_int]
        lib.okf_ref_usable_cores.argtypes = []
        lib.okf_ref_silu_mul.argtypes = [vp, vp, u32, vp]
        lib.okf_ref_silu_mul.restype = None
        lib.okf_ref_add_rmsnorm.argtypes = [vp, vp, vp, vp, u32, u32, ctypes.c_float]
        lib.okf_ref_add_rmsnorm.restype = None
        lib.okf_ref_argmax_rows.argtypes = [vp, u32, u32, vp]
        lib.okf_ref_argmax_rows.restype = None
        _LIB = lib
    return _LIB


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def row_bytes(t: int, n: int) -> int:
    out = ctypes.c_uint64()
    if _lib().okf_ref_row_bytes(t, n, ctypes.byref(out)):
        raise ValueError("bad type/size")
    return out.value


def f16_to_f32(h: int) -> float:
    return _lib().okf_ref_f16_to_f32(h)


def dequant(t: int, row: np.ndarray, n: int) -> np.ndarray:
    row = np.ascontiguousarray(row, np.uint8)
    assert row.size >= row_bytes(t, n)
    out = np.empty(n, np.float32)
    if _lib().okf_ref_dequant(t, _p(row), n, _p(out)):
        raise ValueError("dequant failed")
    return out


def silu_mul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """silu(a) * b, fp32 (the reference's FFN glue)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    assert a.size == b.size
    out = np.empty(a.size, np.float32)
    _lib().okf_ref_silu_mul(_p(a), _p(b), a.size, _p(out))
    return out


def add_rmsnorm(x: np.ndarray, r, w: np.ndarray, eps: float):
    """(x + r, rmsnorm(x + r) * w) per row of x's last axis; r may be None."""
    x = np.array(x, np.float32, order="C", copy=True)
    n = x.shape[-1]
    rows = x.size // n
    rr = None if r is None else np.ascontiguousarray(r, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    assert w.size == n and (rr is None or rr.size == x.size)
    y = np.empty_like(x)
    _lib().okf_ref_add_rmsnorm(_p(x), None if rr is None else _p(rr), _p(w), _p(y), n, rows, eps)
    return x, y


def argmax_rows(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(rows, np.int32)
    _lib().okf_ref_argmax_rows(_p(x), n, rows, _p(out))
    return out


def matvec(t: int, w: np.ndarray, K: int, M: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    assert w.size >= M * row_bytes(t, K) and x.size >= K
    y = np.empty(M, np.float32)
    if _lib().okf_ref_matvec(t, _p(w), K, M, _p(x), _p(y), threads):
        raise ValueError("matvec failed")
    return y


def matmul(t: int, w: np.ndarray, K: int, M: int, X: np.ndarray, threads: int = 0) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    X = np.ascontiguousarray(X, np.float32)
    N = X.size // K
    assert w.size >= M * row_bytes(t, K) and X.size == N * K
    Y = np.empty((N, M), np.float32)
    if _lib().okf_ref_matmul(t, _p(w), K, M, _p(X), N, _p(Y), threads):
        raise ValueError("matmul failed")
    return Y


def usable_cores() -> int:
    return _lib().okf_ref_usable_cores()

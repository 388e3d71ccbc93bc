"""ctypes binding of the C oracle ``imq_oracle.c`` (TEST INFRASTRUCTURE ONLY).

``liboracle.so`` is built by ``oracle/Makefile`` (``build()`` in
``__graft_entry__`` runs it).  Arrays are numpy; bf16 values are uint16 bits.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.oracle_dequantize.argtypes = [p, p, p, p, i64, i64]
        L.oracle_dequantize.restype = ctypes.c_int
        for name in ("oracle_qmm_t", "oracle_qmm_t_f32acc"):
            f = getattr(L, name)
            f.argtypes = [p, p, p, p, p, i64, i64, i64, ctypes.c_int]
            f.restype = ctypes.c_int
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_bf16_to_f32.restype = ctypes.c_float
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f16_to_f32_n.argtypes = [p, p, i64]
        L.oracle_f16_to_f32_n.restype = None
        L.oracle_f32_to_f16_n.argtypes = [p, p, i64]
        L.oracle_f32_to_f16_n.restype = None
        L.oracle_dequantize_t.argtypes = [ctypes.c_int, p, p, p, p, i64, i64]
        L.oracle_dequantize_t.restype = ctypes.c_int
        L.oracle_qmm_t_f64.argtypes = [ctypes.c_int, p, p, p, p, p, i64, i64, i64, ctypes.c_int]
        L.oracle_qmm_t_f64.restype = ctypes.c_int
        L.oracle_max_threads.argtypes = []
        L.oracle_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def dequantize(w: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    biases = np.ascontiguousarray(biases, dtype=np.uint16)
    n, k = w.shape[0], w.shape[1] * 8
    out = np.empty((n, k), dtype=np.uint16)
    rc = lib().oracle_dequantize(_ptr(w), _ptr(scales), _ptr(biases), _ptr(out), n, k)
    if rc != 0:
        raise ValueError(f"oracle_dequantize rejected shape n={n} k={k}")
    return out


def _qmm(fn, x, w, scales, biases, threads):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    biases = np.ascontiguousarray(biases, dtype=np.uint16)
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] * 8 != k:
        raise ValueError("x and w disagree on K")
    y = np.empty((m, n), dtype=np.uint16)
    rc = fn(_ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(y), m, n, k, int(threads))
    if rc != 0:
        raise ValueError(f"oracle qmm rejected shape m={m} n={n} k={k}")
    return y


def qmm_t(x, w, scales, biases, threads: int = 0) -> np.ndarray:
    """bf16 bits RNE_bf16(sum_k x*deq(w)) accumulated in double."""
    return _qmm(lib().oracle_qmm_t, x, w, scales, biases, threads)


def qmm_t_f32acc(x, w, scales, biases, threads: int = 0) -> np.ndarray:
    """f32-accumulating CPU quantized matmul (the timed CPU baseline)."""
    return _qmm(lib().oracle_qmm_t_f32acc, x, w, scales, biases, threads)


def max_threads() -> int:
    return int(lib().oracle_max_threads())


_T_CODES = {"bf16": 0, "f16": 1}


def _t_bits(a: np.ndarray) -> np.ndarray:
    """float16 values or uint16 bit patterns -> contiguous uint16 bits."""
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    return np.ascontiguousarray(a, dtype=np.uint16)


def dequantize_t(w, scales, biases, dtype: str) -> np.ndarray:
    """deq_T(w) [N, K] as T bit patterns (uint16), T = "bf16" or "f16"; scales
    and biases as T bit patterns (f16: float16 arrays are accepted too)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    s, b = _t_bits(scales), _t_bits(biases)
    n, k = w.shape[0], w.shape[1] * 8
    out = np.empty((n, k), dtype=np.uint16)
    rc = lib().oracle_dequantize_t(_T_CODES[dtype], _ptr(w), _ptr(s), _ptr(b), _ptr(out), n, k)
    if rc != 0:
        raise ValueError(f"oracle_dequantize_t rejected dtype={dtype} n={n} k={k}")
    return out


def qmm_t_f64(x, w, scales, biases, dtype: str, threads: int = 0) -> np.ndarray:
    """Unrounded float64 y = x . deq_T(w)^T (sum in k order, in double); x,
    scales, biases as T bit patterns (or float16 arrays for f16)."""
    x, s, b = _t_bits(x), _t_bits(scales), _t_bits(biases)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] * 8 != k:
        raise ValueError("x and w disagree on K")
    y = np.empty((m, n), dtype=np.float64)
    rc = lib().oracle_qmm_t_f64(_T_CODES[dtype], _ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(y),
                                m, n, k, int(threads))
    if rc != 0:
        raise ValueError(f"oracle_qmm_t_f64 rejected dtype={dtype} m={m} n={n} k={k}")
    return y


def f16_to_f32(h) -> np.ndarray:
    """IEEE binary16 bit patterns -> float32 values (the C oracle's widening)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_f16(v) -> np.ndarray:
    """float32 values -> IEEE binary16 bit patterns, RNE (the C oracle's narrowing)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_n(_ptr(v), _ptr(out), v.size)
    return out

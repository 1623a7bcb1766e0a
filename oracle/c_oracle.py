"""ctypes binding of the C oracle (oracle/q4_oracle.c) — TEST INFRASTRUCTURE ONLY.

The C restatement is the fast reference for full-size shapes and the CPU baseline
the benchmark times; it is cross-checked against the numpy restatement in
tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libq4oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    p = ctypes.c_void_p
    i64 = ctypes.c_int64
    ci = ctypes.c_int
    lib.oracle_affine_quantize.argtypes = [p, i64, i64, ci, ci, p, p, p]
    lib.oracle_affine_dequantize.argtypes = [p, p, p, i64, i64, ci, ci, p]
    lib.oracle_qmm_f64.argtypes = [p, i64, i64, p, p, p, i64, ci, ci, p]
    lib.oracle_qmm_f32.argtypes = [p, i64, i64, p, p, p, i64, ci, ci, p, ci]
    for f in (lib.oracle_affine_quantize, lib.oracle_affine_dequantize, lib.oracle_qmm_f64,
              lib.oracle_qmm_f32, lib.oracle_max_threads):
        f.restype = ci
    _lib = lib
    return lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def quantize(w: np.ndarray, group_size: int = 64, bits: int = 4):
    lib = load()
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    wq = np.zeros((n, k * bits // 32), dtype=np.uint32)
    s = np.zeros((n, k // group_size), dtype=np.uint16)
    b = np.zeros((n, k // group_size), dtype=np.uint16)
    if lib.oracle_affine_quantize(_ptr(w), n, k, group_size, bits, _ptr(wq), _ptr(s), _ptr(b)) != 0:
        raise ValueError("oracle_affine_quantize rejected its arguments")
    return wq, s, b


def dequantize(wq, scales, biases, group_size: int = 64, bits: int = 4) -> np.ndarray:
    lib = load()
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    b = np.ascontiguousarray(biases, dtype=np.uint16)
    n = wq.shape[0]
    k = wq.shape[1] * 32 // bits
    out = np.empty((n, k), dtype=np.float32)
    if lib.oracle_affine_dequantize(_ptr(wq), _ptr(s), _ptr(b), n, k, group_size, bits, _ptr(out)) != 0:
        raise ValueError("oracle_affine_dequantize rejected its arguments")
    return out


def qmm_f64(x_bits, wq, scales, biases, group_size: int = 64, bits: int = 4) -> np.ndarray:
    lib = load()
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    b = np.ascontiguousarray(biases, dtype=np.uint16)
    m, k = x.shape
    n = wq.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    if lib.oracle_qmm_f64(_ptr(x), m, k, _ptr(wq), _ptr(s), _ptr(b), n, group_size, bits, _ptr(y)) != 0:
        raise ValueError("oracle_qmm_f64 rejected its arguments")
    return y


def qmm_f32(x_bits, wq, scales, biases, group_size: int = 64, bits: int = 4, threads: int = 0,
            out: np.ndarray | None = None) -> np.ndarray:
    lib = load()
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    m, k = x.shape
    n = wq.shape[0]
    y = out if out is not None else np.empty((m, n), dtype=np.float32)
    if lib.oracle_qmm_f32(_ptr(x), m, k, _ptr(wq), _ptr(scales), _ptr(biases), n, group_size, bits,
                          _ptr(y), threads) != 0:
        raise ValueError("oracle_qmm_f32 rejected its arguments")
    return y


def max_threads() -> int:
    return int(load().oracle_max_threads())

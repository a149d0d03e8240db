"""ctypes wrapper over oracle/libdk_oracle.so (the scalar C restatement).

TEST INFRASTRUCTURE ONLY (imported by tests/ as a checker).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libdk_oracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        i64, P = ctypes.c_int64, ctypes.c_void_p
        L.dko_f32_to_f16.restype = ctypes.c_uint16
        L.dko_f32_to_f16.argtypes = [ctypes.c_float]
        L.dko_f16_to_f32.restype = ctypes.c_float
        L.dko_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.dko_quantize_pack.restype = ctypes.c_int
        L.dko_quantize_pack.argtypes = [P, i64, i64, P, P]
        L.dko_unpack.restype = None
        L.dko_unpack.argtypes = [P, i64, i64, P]
        L.dko_gemv_f64.restype = None
        L.dko_gemv_f64.argtypes = [P, P, P, i64, i64, i64, P]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f32_to_f16_bits(v: float) -> int:
    return int(lib().dko_f32_to_f16(ctypes.c_float(v)))


def quantize_and_pack(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = w.shape
    packed = np.zeros((m, k // 8), dtype=np.int32)
    scales = np.zeros((m, k // 128), dtype=np.uint16)
    rc = lib().dko_quantize_pack(_ptr(w), m, k, _ptr(packed), _ptr(scales))
    if rc != 0:
        raise ValueError("K must be a multiple of 128")
    return packed, scales.view(np.float16)


def unpack_to_int(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed).view(np.int32)
    m, words = packed.shape
    q = np.zeros((m, words * 8), dtype=np.int32)
    lib().dko_unpack(_ptr(packed), m, words * 8, _ptr(q))
    return q


def gemv_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float16).view(np.uint16)
    packed = np.ascontiguousarray(packed).view(np.int32)
    scales = np.ascontiguousarray(scales, dtype=np.float16).view(np.uint16)
    m, words = packed.shape
    k = words * 8
    b = x.shape[0]
    y = np.zeros((b, m), dtype=np.float64)
    lib().dko_gemv_f64(_ptr(packed), _ptr(scales), _ptr(x), m, k, b, _ptr(y))
    return y

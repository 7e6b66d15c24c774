"""ctypes loader for oracle/liboracle.so (test infrastructure only)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_rns_matmul_centered.restype = ctypes.c_int
        lib.oracle_rns_matmul_centered.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        _lib = lib
    return _lib


def rns_matmul_centered(a: np.ndarray, b: np.ndarray, moduli) -> np.ndarray:
    """Centered RNS product of int8 a [M, K] and b [K, N] -> int64 [M, N]."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    mods = np.ascontiguousarray(moduli, dtype=np.int32)
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError("K dimensions do not match")
    out = np.empty((m, n), dtype=np.int64)
    rc = load().oracle_rns_matmul_centered(
        a.ctypes.data, b.ctypes.data, m, k, n, mods.ctypes.data, len(mods),
        out.ctypes.data)
    if rc != 0:
        raise RuntimeError("oracle_rns_matmul_centered failed")
    return out

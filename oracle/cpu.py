"""ctypes wrapper of ``oracle/c/liboracle_cpu.so`` — the C/OpenMP restatement of the oracle GEMV, used as the timed
CPU baseline and cross-checked against the numpy oracle (test infrastructure only)."""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent / "c"
_LIB = _DIR / "liboracle_cpu.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        if not _LIB.exists():
            build()
        _lib = C.CDLL(str(_LIB))
        f = C.c_void_p
        _lib.oracle_nvfp4_gemv.argtypes = [f, f, C.c_float, f, C.c_int, C.c_int, C.c_int, f, C.c_int]
        _lib.oracle_int4_gemv.argtypes = [f, f, f, f, C.c_int, C.c_int, C.c_int, f, C.c_int]
    return _lib


def threads() -> int:
    return len(os.sched_getaffinity(0))


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def nvfp4_gemv(m: dict, x: np.ndarray, nthreads: int | None = None) -> np.ndarray:
    """``x @ Wᵀ`` for an oracle NVFP4 dict (``weight``, ``weight_scale``, ``weight_scale_2``); ``x [M, K]``, M ≤ 16."""
    codes = np.ascontiguousarray(m["weight"], np.uint8)
    sc = np.ascontiguousarray(m["weight_scale"], np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    n, k = codes.shape[0], codes.shape[1] * 2
    y = np.empty((x.shape[0], n), np.float32)
    lib().oracle_nvfp4_gemv(_p(codes), _p(sc), float(m["weight_scale_2"]), _p(x), x.shape[0], n, k, _p(y),
                            nthreads or threads())
    return y


def int4_gemv(m: dict, x: np.ndarray, nthreads: int | None = None) -> np.ndarray:
    codes = np.ascontiguousarray(m["weight"], np.uint8)
    sc = np.ascontiguousarray(m["scales"], np.float32)
    bi = np.ascontiguousarray(m["biases"], np.float32)
    x = np.ascontiguousarray(x, np.float32)
    n, k = codes.shape[0], codes.shape[1] * 2
    y = np.empty((x.shape[0], n), np.float32)
    lib().oracle_int4_gemv(_p(codes), _p(sc), _p(bi), _p(x), x.shape[0], n, k, _p(y), nthreads or threads())
    return y
